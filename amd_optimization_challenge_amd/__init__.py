"""MI355X (gfx950) MLA absorbed-decode operator.

Public surface:
  custom_kernel(data)  -- drop-in for mixed-mla/submission.py:custom_kernel
  ops                  -- per-stage wrappers of libmla_mi355x.so
  inputs               -- seeded inputs in the reference's tuple layout
"""
from .submission import custom_kernel  # noqa: F401

__all__ = ["custom_kernel"]
