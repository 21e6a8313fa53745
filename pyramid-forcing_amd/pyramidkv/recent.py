from .base import RecentStrategy  # noqa: F401
