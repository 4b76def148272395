"""Linear parameter-varying recurrences (philtorch.lpv)."""
from .recur import linear_recurrence  # noqa: F401
