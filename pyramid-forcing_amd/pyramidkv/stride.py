from .base import StrideStrategy  # noqa: F401
