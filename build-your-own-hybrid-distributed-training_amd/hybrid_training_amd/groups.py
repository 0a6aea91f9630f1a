"""Group handles as the hot path sees them: a size and this rank's position.

The flat-parameter layout, the AVG pre-divide and the norm weighting depend only
on a group's size and on the rank's index in it.  :class:`GroupHandle` keeps the
fields of ``distributed/groups.py:78-144`` of the reference so objects built for
it carry over; no process group is ever used, because this library issues no
collectives.  :meth:`GroupHandle.local_view` describes rank ``r`` of a ``G``-rank
group for a single device that holds that rank's share of the work.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

from .errors import CollectiveError, format_error

__all__ = ["GroupHandle"]


@dataclass(frozen=True)
class GroupHandle:
    """A named group of ranks and this rank's place in it."""

    name: str
    ranks: tuple[int, ...]
    local_rank: int
    global_rank: int
    process_group: Any = None

    def __post_init__(self) -> None:
        if not self.ranks or not 0 <= self.local_rank < len(self.ranks):
            raise CollectiveError(
                format_error(
                    "groups.GroupHandle",
                    "the local rank must index the group's rank list",
                    expected=f"0 <= local_rank < {len(self.ranks)}",
                    observed=self.local_rank,
                    resolution="build the handle from the group's real membership",
                )
            )

    @property
    def size(self) -> int:
        """How many ranks the group spans."""
        return len(self.ranks)

    @property
    def is_trivial(self) -> bool:
        """True for a one-member group, where every collective is the identity."""
        return len(self.ranks) == 1

    @property
    def source_rank(self) -> int:
        """Global rank of the group's broadcast source."""
        return self.ranks[0]

    @classmethod
    def trivial(cls, name: str = "trivial", rank: int = 0) -> GroupHandle:
        """One-member group with no backend communicator (``groups.py:121-144``)."""
        return cls(name=name, ranks=(rank,), local_rank=0, global_rank=rank, process_group=None)

    @classmethod
    def local_view(cls, name: str, size: int, rank: int) -> GroupHandle:
        """Rank ``rank`` of a ``size``-rank group, laid out on this device alone."""
        if size < 1:
            raise CollectiveError(
                format_error("groups.GroupHandle.local_view", "group size must be positive",
                             expected=">= 1", observed=size)
            )
        return cls(name=name, ranks=tuple(range(size)), local_rank=rank, global_rank=rank)

    def __repr__(self) -> str:
        return (
            f"GroupHandle(name={self.name!r}, size={self.size}, "
            f"local_rank={self.local_rank}, ranks={self.ranks})"
        )
