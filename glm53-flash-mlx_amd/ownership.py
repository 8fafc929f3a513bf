"""Storage-lifetime contracts for tensors that a resident structure keeps.

Counterpart of the reference's glm53_flash_mlx/ownership.py:13-198 (same
names, categories and errors, since ``PackedFP8ExpertBank`` takes these
leases at its boundary).  A resident structure -- an expert bank whose
device pointers are recorded by native plans and captured HIP graphs --
may keep storage it owns, or storage borrowed from an owner that it keeps
alive; it must never keep a borrowed-ephemeral buffer (a staging copy that
its producer may reuse), which has to be copied into owned storage first.

Here the values are torch tensors (device or host); "row-major contiguous"
means ``Tensor.is_contiguous()``, and an owned copy is a fresh contiguous
clone on the same device.
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
    """A storage lifetime that cannot back a resident structure."""


def _needs_owner(ownership: TensorOwnership, owner) -> None:
    if ownership is TensorOwnership.BORROWED_STABLE and owner is None:
        raise TensorOwnershipError("borrowed-stable storage requires an owner retained for its lifetime")


@dataclass(frozen=True)
class TensorLease:
    """A tensor together with the lifetime its holder promises."""

    value: torch.Tensor
    ownership: TensorOwnership
    layout: TensorLayout = TensorLayout.UNKNOWN
    owner: object | None = None

    def __post_init__(self) -> None:
        _needs_owner(self.ownership, self.owner)


@dataclass(frozen=True)
class ResidentTensor:
    """A lease that a resident structure may keep: never ephemeral, always
    row-major contiguous, and a borrowed one keeps its owner referenced."""

    value: torch.Tensor
    ownership: TensorOwnership
    layout: TensorLayout
    owner: object | None = None

    def __post_init__(self) -> None:
        if self.ownership is TensorOwnership.BORROWED_EPHEMERAL:
            raise TensorOwnershipError("resident structures cannot retain borrowed-ephemeral storage")
        if self.layout is not TensorLayout.ROW_MAJOR_CONTIGUOUS:
            raise TensorOwnershipError("resident tensors require the row-major contiguous layout contract")
        if self.ownership is TensorOwnership.BORROWED_STABLE and self.owner is None:
            raise TensorOwnershipError("borrowed-stable resident storage must retain its owner")


def owned_tensor(value: torch.Tensor, *, layout: TensorLayout = TensorLayout.UNKNOWN) -> TensorLease:
    """Storage this runtime created and controls the lifetime of."""
    return TensorLease(value, TensorOwnership.OWNED, layout)


def borrowed_stable_tensor(value: torch.Tensor, *, owner: object,
                           layout: TensorLayout = TensorLayout.UNKNOWN) -> TensorLease:
    """Storage of `owner`, which stays referenced as long as the lease is kept."""
    return TensorLease(value, TensorOwnership.BORROWED_STABLE, layout, owner)


def borrowed_ephemeral_tensor(value: torch.Tensor, *, owner: object | None = None,
                              layout: TensorLayout = TensorLayout.UNKNOWN) -> TensorLease:
    """Staging storage that its producer may reuse once the load step ends."""
    return TensorLease(value, TensorOwnership.BORROWED_EPHEMERAL, layout, owner)


def _contiguous(value: torch.Tensor) -> torch.Tensor:
    return value if value.is_contiguous() else value.contiguous()


def require_resident(lease: TensorLease | ResidentTensor) -> ResidentTensor:
    """Admit a lease at a resident boundary.  Never copies behind the
    caller's back: an ephemeral lease is refused (copy it with
    materialize_owned first), a bare tensor has no contract and is refused."""
    if isinstance(lease, ResidentTensor):
        return lease
    if not isinstance(lease, TensorLease):
        raise TypeError("resident tensors require an explicit TensorLease; bare arrays have no storage "
                        "lifetime contract")
    if lease.ownership is TensorOwnership.BORROWED_EPHEMERAL:
        raise TensorOwnershipError("borrowed-ephemeral storage must call materialize_owned() before crossing a "
                                   "resident boundary")
    return ResidentTensor(_contiguous(lease.value), lease.ownership, TensorLayout.ROW_MAJOR_CONTIGUOUS, lease.owner)


def materialize_owned(lease: TensorLease | ResidentTensor) -> ResidentTensor:
    """Owned storage that shares nothing with any borrowed source."""
    if not isinstance(lease, (TensorLease, ResidentTensor)):
        raise TypeError("materialize_owned() requires an explicit storage contract")
    if lease.ownership is TensorOwnership.OWNED:
        value = _contiguous(lease.value)
    else:
        value = lease.value.clone(memory_format=torch.contiguous_format)
    return ResidentTensor(value, TensorOwnership.OWNED, TensorLayout.ROW_MAJOR_CONTIGUOUS)


def resident_concatenate(leases: Iterable[TensorLease | ResidentTensor], *, axis: int) -> ResidentTensor:
    """One owned tensor joined from resident-admissible sources."""
    parts = [require_resident(lease).value for lease in leases]
    if not parts:
        raise ValueError("cannot concatenate an empty resident tensor list")
    return ResidentTensor(torch.cat(parts, dim=axis).contiguous(), TensorOwnership.OWNED,
                          TensorLayout.ROW_MAJOR_CONTIGUOUS)


def storage_descriptor(value: TensorLease | ResidentTensor) -> dict[str, str]:
    return {"ownership": value.ownership.value, "layout": value.layout.value}
