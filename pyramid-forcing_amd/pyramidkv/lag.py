from .base import LagStrategy  # noqa: F401
