"""Linear time-invariant recurrences, state-space models and filters (philtorch.lti)."""
from .recur import LTIRecurrence, linear_recurrence  # noqa: F401
from .ssm import LTIMatrixRecurrence, diag_state_space, state_space, state_space_recursion  # noqa: F401
from .filtering import filtfilt, lfilter, lfilter_zi, sosfilt  # noqa: F401
