"""Linear parameter-varying recurrences and state-space models (philtorch.lpv)."""
from .recur import linear_recurrence  # noqa: F401
from .ssm import MatrixRecurrence, state_space, state_space_recursion  # noqa: F401
