from .base import CyclicStrategy  # noqa: F401
