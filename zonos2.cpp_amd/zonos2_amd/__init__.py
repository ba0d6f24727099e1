"""Python host mirror of the MI355X decode-step library (ctypes over include/z2h.h)."""
from .configs import ModelConfig, Workload  # noqa: F401
