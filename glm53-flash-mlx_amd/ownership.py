"""Storage leases for tensors that a resident structure keeps.

A resident structure -- an expert bank whose device addresses native plans
and captured HIP graphs record -- has to know, for every tensor it keeps,
whose storage it is and how long that storage lives.  A lease says so, in
one of three categories:

* ``owned``: this runtime allocated the storage and decides when it dies;
  the structure may keep it and rewrite it (a bank re-lays owned weights in
  place);
* ``borrowed-stable``: another object owns the storage and outlives the
  lease; the lease keeps a reference to that owner, and the structure never
  writes the storage;
* ``borrowed-ephemeral``: a staging buffer its producer may overwrite once
  the load step ends; a structure never keeps one -- it is copied into owned
  storage first (``materialize_owned``).

Leases are values, checked when built; admission at a resident boundary
(``require_resident``) turns a lease into a ``ResidentTensor`` and never
copies on its own.  The names, the category and layout strings and
``storage_descriptor`` follow the reference runtime's ownership module
(glm53_flash_mlx/ownership.py:13-198), because ``PackedFP8ExpertBank`` takes
these leases at its constructor (packed.py:750-787) and reports their
descriptors.  Values are torch tensors on any device.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum
from typing import Iterable

import torch


class TensorOwnership(str, Enum):
    OWNED = "owned"
    BORROWED_STABLE = "borrowed-stable"
    BORROWED_EPHEMERAL = "borrowed-ephemeral"


class TensorLayout(str, Enum):
    UNKNOWN = "unknown"
    ROW_MAJOR_CONTIGUOUS = "row-major-contiguous"


class TensorOwnershipError(ValueError):
    """A lease whose lifetime a resident structure cannot rely on."""


# What each category needs, checked in one place: (an owner reference is
# required, a resident structure may keep it, a resident structure may
# rewrite it).
_RULES = {
    TensorOwnership.OWNED: (False, True, True),
    TensorOwnership.BORROWED_STABLE: (True, True, False),
    TensorOwnership.BORROWED_EPHEMERAL: (False, False, False),
}


def _check_owner(ownership: TensorOwnership, owner) -> None:
    needs_owner = _RULES[TensorOwnership(ownership)][0]
    if needs_owner and owner is None:
        raise TensorOwnershipError(
            f"a {TensorOwnership(ownership).value} lease names no owner: the object that frees the storage must be "
            "given so the lease can keep it alive")


@dataclass(frozen=True)
class TensorLease:
    """A tensor and the lifetime promised for its storage."""

    value: torch.Tensor
    ownership: TensorOwnership
    layout: TensorLayout = TensorLayout.UNKNOWN
    owner: object | None = None

    def __post_init__(self) -> None:
        _check_owner(self.ownership, self.owner)

    @property
    def writable(self) -> bool:
        """Whether a structure holding this lease may rewrite the storage."""
        return _RULES[self.ownership][2]


@dataclass(frozen=True)
class ResidentTensor:
    """An admitted lease: keepable (owned or borrowed-stable), contiguous in
    row-major order, and, when borrowed, holding its owner."""

    value: torch.Tensor
    ownership: TensorOwnership
    layout: TensorLayout
    owner: object | None = None

    def __post_init__(self) -> None:
        if not _RULES[TensorOwnership(self.ownership)][1]:
            raise TensorOwnershipError(
                f"{TensorOwnership(self.ownership).value} storage cannot be resident: copy it with "
                "materialize_owned() first")
        if self.layout is not TensorLayout.ROW_MAJOR_CONTIGUOUS:
            raise TensorOwnershipError(
                f"a resident tensor is row-major contiguous by contract; got layout '{self.layout.value}'")
        _check_owner(self.ownership, self.owner)

    @property
    def writable(self) -> bool:
        return _RULES[self.ownership][2]


def owned_tensor(value: torch.Tensor, *, layout: TensorLayout = TensorLayout.UNKNOWN) -> TensorLease:
    """Lease on storage this runtime allocated."""
    return TensorLease(value, TensorOwnership.OWNED, layout)


def borrowed_stable_tensor(value: torch.Tensor, *, owner: object,
                           layout: TensorLayout = TensorLayout.UNKNOWN) -> TensorLease:
    """Lease on storage of `owner`, which the lease keeps referenced."""
    return TensorLease(value, TensorOwnership.BORROWED_STABLE, layout, owner)


def borrowed_ephemeral_tensor(value: torch.Tensor, *, owner: object | None = None,
                              layout: TensorLayout = TensorLayout.UNKNOWN) -> TensorLease:
    """Lease on a staging buffer its producer may reuse after the load step."""
    return TensorLease(value, TensorOwnership.BORROWED_EPHEMERAL, layout, owner)


def _admit(value: torch.Tensor, ownership: TensorOwnership, owner, *, copy: bool) -> ResidentTensor:
    """The one place a tensor becomes resident: a private contiguous copy
    when `copy` (owned from then on), else the tensor itself made
    contiguous (which copies only a strided view)."""
    if copy:
        return ResidentTensor(value.clone(memory_format=torch.contiguous_format), TensorOwnership.OWNED,
                              TensorLayout.ROW_MAJOR_CONTIGUOUS)
    return ResidentTensor(value.contiguous(), ownership, TensorLayout.ROW_MAJOR_CONTIGUOUS, owner)


def _lease_of(lease, who: str) -> TensorLease | ResidentTensor:
    if not isinstance(lease, (TensorLease, ResidentTensor)):
        raise TypeError(f"{who} takes a TensorLease (owned_tensor / borrowed_stable_tensor / "
                        f"borrowed_ephemeral_tensor), not a bare {type(lease).__name__}: a bare tensor states "
                        "no storage lifetime")
    return lease


def require_resident(lease: TensorLease | ResidentTensor) -> ResidentTensor:
    """Admit a lease at a resident boundary without copying its data: an
    ephemeral lease is refused (materialize_owned makes the copy), a bare
    tensor is refused (it has no lifetime contract)."""
    lease = _lease_of(lease, "require_resident()")
    if isinstance(lease, ResidentTensor):
        return lease
    if not _RULES[lease.ownership][1]:
        raise TensorOwnershipError(
            "a borrowed-ephemeral tensor may be overwritten by its producer; call materialize_owned() on it "
            "before handing it to a resident structure")
    return _admit(lease.value, lease.ownership, lease.owner, copy=False)


def materialize_owned(lease: TensorLease | ResidentTensor) -> ResidentTensor:
    """Owned storage sharing nothing with a borrowed source: an owned lease
    is admitted as it is, any borrowed one is copied."""
    lease = _lease_of(lease, "materialize_owned()")
    borrowed = lease.ownership is not TensorOwnership.OWNED
    if isinstance(lease, ResidentTensor) and not borrowed:
        return lease
    return _admit(lease.value, TensorOwnership.OWNED, None, copy=borrowed)


def resident_concatenate(leases: Iterable[TensorLease | ResidentTensor], *, axis: int) -> ResidentTensor:
    """Join keepable sources along `axis` into new owned storage."""
    values = [require_resident(lease).value for lease in leases]
    if len(values) == 0:
        raise ValueError("resident_concatenate() got no tensors to join")
    return _admit(torch.cat(values, dim=axis), TensorOwnership.OWNED, None, copy=False)


def storage_descriptor(value: TensorLease | ResidentTensor) -> dict[str, str]:
    """{"ownership": category, "layout": layout} of a lease, as strings."""
    return {"ownership": TensorOwnership(value.ownership).value, "layout": TensorLayout(value.layout).value}
