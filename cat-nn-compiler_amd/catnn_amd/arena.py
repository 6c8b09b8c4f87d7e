"""First-fit arena planning: `place_arena` and `arena_conflict`
(crates/catnn-compile/src/schedule.rs:61-136), computed by the backend
library on the host.  The device program uses the same planner for its
activation buffers."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

from ._lib import CArenaAlloc, CBufferReq, check, lib


@dataclass
class BufferReq:
    """`BufferReq` (schedule.rs:61-70); lifetimes are inclusive ticks."""
    id: str
    bytes: int
    live_from: int
    live_to: int
    checkpoint: bool = False


@dataclass
class ArenaAlloc:
    """`ArenaAlloc` (schedule.rs:36-43)."""
    id: str
    bytes: int
    offset: int
    live_from: int
    live_to: int


def place_arena(reqs: Sequence[BufferReq], cap: int) -> List[ArenaAlloc]:
    """Raises CatError(Fibration) naming the buffer that overflows `cap`."""
    n = len(reqs)
    ids = [r.id.encode() for r in reqs]
    creqs = (CBufferReq * max(n, 1))()
    for i, r in enumerate(reqs):
        creqs[i].id = ids[i]
        creqs[i].bytes = r.bytes
        creqs[i].live_from = r.live_from
        creqs[i].live_to = r.live_to
        creqs[i].checkpoint = int(r.checkpoint)
    out = (CArenaAlloc * max(n, 1))()
    check(lib.catnn_place_arena(creqs, n, cap, out))
    return [ArenaAlloc(a.id.decode(), a.bytes, a.offset, a.live_from, a.live_to) for a in out[:n]]


def arena_conflict(allocs: Sequence[ArenaAlloc]) -> Optional[Tuple[str, str]]:
    n = len(allocs)
    arr = (CArenaAlloc * max(n, 1))()
    for i, a in enumerate(allocs):
        arr[i].id = a.id.encode()[:127]
        arr[i].bytes = a.bytes
        arr[i].offset = a.offset
        arr[i].live_from = a.live_from
        arr[i].live_to = a.live_to
    c, i, j = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    check(lib.catnn_arena_conflict(arr, n, ctypes.byref(c), ctypes.byref(i), ctypes.byref(j)))
    if not c.value:
        return None
    return allocs[i.value].id, allocs[j.value].id
