"""The package's argument-error type.

``ContractError`` is what the reference raises when inputs do not satisfy
its native contract (``contract.py:54-55``): shapes, ranges and layouts that
the path does not accept.  Every host-side check in this package raises it
(or a subclass) rather than letting a bad argument reach the HIP library.
"""

from __future__ import annotations


class ContractError(ValueError):
    """The inputs do not satisfy what the MoE path accepts."""
