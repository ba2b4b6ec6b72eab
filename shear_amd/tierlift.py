"""TierLift: the bounded host reducer of the edge-record stream.

Host mirror of SpillEdgeSink feeding ExternalHashPruneReducer (paths relative
to shear-core/src/algorithm/pipnn/spill_hashprune.rs): records routed to
source-range shards (:569-651), buffered on the host up to a budget and past
it written as src-sorted segments to part files with a segment manifest
(:727-851), then reduced shard by shard (:853-892).  The work runs in
libtessa_hip.so (``tessa_tierlift_*``): records leave the device through
two pinned staging slots on a side stream while the caller's stream goes on,
a native worker routes and spills them, and the reservoir merge at the end
runs on the GPU shard by shard.  Spill files are readable with
``spill.read_spill_artifacts``.
"""
from __future__ import annotations

import collections
import ctypes as C
from dataclasses import dataclass

import torch

from . import _native as N
from .tessa import _ptr, _stream_ptr

DEFAULT_SHARD_POINTS = 1_000_000  # spill_hashprune.rs:26
DEFAULT_STAGING_RECORDS = 1 << 24  # 256 MiB per pinned slot


@dataclass
class TierLiftParams:
    host_budget_bytes: int
    spill_base: str | None = None       # candidate path: spill files go next to it, named after its stem
    shard_points: int = DEFAULT_SHARD_POINTS
    staging_records: int = DEFAULT_STAGING_RECORDS
    threads: int = 0                     # host threads for routing and spill sorting (0: up to 16)
    expected_records: int = 0            # about how many records will be pushed (0: unknown)


class TierLiftReducer:
    """Reservoirs of points [0, num_points), fed from device records through
    host memory bounded by ``params.host_budget_bytes``."""

    def __init__(self, num_points: int, l_max: int, params: TierLiftParams, device="cuda"):
        self.num_points = int(num_points)
        self.l_max = int(l_max)
        self.device = torch.device(device)
        self._lib = N.load()
        self._base = params.spill_base.encode() if params.spill_base else None
        cfg = N.TierLiftConfig(self.num_points, int(params.shard_points), int(params.host_budget_bytes),
                               int(params.staging_records), self._base, self.l_max, int(params.threads),
                               int(params.expected_records))
        h = C.c_void_p()
        with torch.cuda.device(self.device):
            N.check(self._lib.tessa_tierlift_create(C.byref(cfg), C.byref(h)), "tierlift create")
        self._h = h
        self._inflight: collections.deque = collections.deque()  # (seq, tensor) until copied
        self.stats: dict = {}

    def close(self) -> None:
        if self._h:
            N.check(self._lib.tessa_tierlift_destroy(self._h), "tierlift destroy")
            self._h = C.c_void_p()
        self._inflight.clear()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _release(self) -> None:
        seq = C.c_uint64()
        N.check(self._lib.tessa_tierlift_copied(self._h, C.byref(seq)), "tierlift copied")
        while self._inflight and self._inflight[0][0] <= seq.value:
            self._inflight.popleft()

    def push(self, records: torch.Tensor, count: int | None = None, stream: torch.cuda.Stream | None = None) -> int:
        """Queue the first ``count`` rows of a device int32 [n, 4] record tensor
        (as ``edges.emit_edge_records`` writes it).  The tensor is held until
        its copy has completed; returns the batch's sequence number."""
        if records.dtype != torch.int32 or records.dim() != 2 or records.shape[1] != 4:
            raise ValueError("records must be an int32 [n, 4] tensor (16-byte SpillRecord16 rows)")
        n = records.shape[0] if count is None else int(count)
        if n > records.shape[0]:
            raise ValueError(f"count {n} exceeds the {records.shape[0]} records given")
        if n == 0:
            return 0
        seq = C.c_uint64()
        N.check(self._lib.tessa_tierlift_push(self._h, _ptr(records), n, _stream_ptr(stream), C.byref(seq)),
                "tierlift push")
        self._inflight.append((seq.value, records))
        self._release()
        return seq.value

    def wait(self, seq: int) -> None:
        N.check(self._lib.tessa_tierlift_wait(self._h, int(seq)), "tierlift wait")
        self._release()

    def finish(self, stream: torch.cuda.Stream | None = None):
        """(targets int32 [num_points, l_max], counts int32 [num_points]) after
        reducing every pushed record; ``self.stats`` holds the reducer's
        counters (records, spilled bytes, segments, host peak, times)."""
        t = torch.empty((self.num_points, self.l_max), dtype=torch.int32, device=self.device)
        c = torch.empty(self.num_points, dtype=torch.int32, device=self.device)
        st = N.TierLiftStats()
        N.check(self._lib.tessa_tierlift_finish(self._h, _ptr(t), _ptr(c), _stream_ptr(stream), C.byref(st)),
                "tierlift finish")
        self._inflight.clear()
        self.stats = st.as_dict()
        return t, c
