from .base import MergeStrategy  # noqa: F401
