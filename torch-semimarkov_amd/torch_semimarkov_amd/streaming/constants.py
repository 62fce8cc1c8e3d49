"""Shared constants (reference ``streaming/constants.py:10``)."""

#: Sentinel for unreachable log-space states; the reference uses -1e9, not -inf.
NEG_INF = -1e9
