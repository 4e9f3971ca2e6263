"""Contract errors (the reference's ``contract.py:54-55``)."""

from __future__ import annotations


class ContractError(ValueError):
    """The inputs do not satisfy the supported native contract."""
