"""Linear time-invariant recurrences and filters (philtorch.lti)."""
from .recur import LTIRecurrence, linear_recurrence  # noqa: F401
