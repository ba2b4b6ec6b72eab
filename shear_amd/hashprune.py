"""HashPrune reservoirs on the GPU: the consumer of the edge-record stream.

Host mirror of the reference's reducer side (paths relative to
shear-core/src/algorithm/pipnn/):

* ``HashPruneReducer``                 HashPruneReservoir per point (hash_prune.rs:266-280,
  insert :1243-1246 / :1333-1453) driven as ExternalHashPruneReducer drives it
  (spill_hashprune.rs:853-936, per-edge insert :2686-2719, emit :3203-3221)
* ``reduce_spill_records_ordered``     ExternalHashPruneReducer::reduce_spill_artifacts_ordered
  (spill_hashprune.rs:875-892): one neighbour list per point, slot order

* ``HashPruneBackfill``                the named R-half backfill policies (PiPNNParams
  hashprune_backfill_mode rhalf-* with hashprune_rhalf_hash_quota,
  hashprune_rhalf_max_backfill_per_row, hashprune_soft_tier_priority_alpha:
  params.rs:2070-2083, validated as :2696-2729); ``PRODUCTION_BACKFILL`` is
  the build_shear_index binary's default (SoftTier-Q3, alpha 1.02, 3 per row,
  apps/build_shear_index/src/main.rs:2360-2374)

Without a policy, backfill and evidence are off (PiPNNParams' defaults,
params.rs:3346-3350).  The reservoirs live in device memory (libtessa_hip.so,
``tessa_hashprune_*``); records are merged batch by batch in any order, with
or without a policy (its result is the reference's order-independent
characterization, hash_prune.rs:2601-2682).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _native as N
from .edges import EDGE_RECORD_DTYPE
from .tessa import _ptr, _stream_ptr

DEFAULT_L_MAX = 64  # params.rs:3346

# PiPNNHashPruneBackfillMode names (params.rs:1935-1966) of the named R-half
# policies, as tessa_hashprune_backfill.mode numbers them
BACKFILL_MODES = {"off": 0, "rhalf-hash-slot-1": 1, "rhalf-distance-first-q3": 2, "rhalf-soft-tier-q3": 3,
                  "rhalf-hard-tier-q3": 4}


@dataclass(frozen=True)
class HashPruneBackfill:
    """A named R-half policy; None fields take the reference's defaults
    (hash_prune_backfill.rs:44-83: quota 1 for rhalf-hash-slot-1, else 3;
    SoftTier alpha 1.1; per-row cap floor(l_max / 2))."""
    mode: str = "off"
    hash_quota: int | None = None
    max_backfill_per_row: int | None = None
    soft_tier_priority_alpha: float | None = None

    def native(self) -> N.HashPruneBackfill:
        if self.mode not in BACKFILL_MODES:
            raise ValueError(f"unsupported hashprune_backfill_mode {self.mode!r} "
                             f"(the named R-half policies: {', '.join(BACKFILL_MODES)})")
        return N.HashPruneBackfill(BACKFILL_MODES[self.mode], int(self.hash_quota or 0),
                                   int(self.max_backfill_per_row or 0), float(self.soft_tier_priority_alpha or 0.0))


# build_shear_index's apply_production_hashprune_defaults (main.rs:2360-2374)
PRODUCTION_BACKFILL = HashPruneBackfill("rhalf-soft-tier-q3", None, 3, 1.02)


class HashPruneReducer:
    """Device-resident HashPrune reservoirs for points [0, num_points)."""

    def __init__(self, num_points: int, l_max: int = DEFAULT_L_MAX, device="cuda",
                 backfill: HashPruneBackfill | None = None):
        self.num_points = int(num_points)
        self.l_max = int(l_max)
        self.device = torch.device(device)
        self.backfill = backfill if backfill is not None and backfill.mode != "off" else None
        self._lib = N.load()
        h = C.c_void_p()
        with torch.cuda.device(self.device):
            if self.backfill is None:
                st = self._lib.tessa_hashprune_create(self.num_points, self.l_max, C.byref(h))
            else:
                pol = self.backfill.native()
                st = self._lib.tessa_hashprune_create_backfill(self.num_points, self.l_max, C.byref(pol), C.byref(h))
            N.check(st, "hashprune create")
        self._h = h

    def close(self) -> None:
        if self._h:
            N.check(self._lib.tessa_hashprune_destroy(self._h), "hashprune destroy")
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def insert(self, records, count: int | None = None, stream: torch.cuda.Stream | None = None) -> None:
        """Merge SpillRecord16 records: a device int32 [n, 4] tensor (as written
        by ``edges.emit_edge_records``; the first ``count`` rows) or a host
        EDGE_RECORD_DTYPE array (uploaded first).  Synchronises the stream."""
        if isinstance(records, np.ndarray):
            raw = np.ascontiguousarray(records, EDGE_RECORD_DTYPE).view(np.uint8).view(np.int32).reshape(-1, 4)
            records = torch.from_numpy(raw.copy()).to(self.device)
        if records.dtype != torch.int32 or records.dim() != 2 or records.shape[1] != 4:
            raise ValueError("records must be an int32 [n, 4] tensor (16-byte SpillRecord16 rows)")
        n = records.shape[0] if count is None else int(count)
        if n > records.shape[0]:
            raise ValueError(f"count {n} exceeds the {records.shape[0]} records given")
        N.check(self._lib.tessa_hashprune_insert(self._h, _ptr(records), n, _stream_ptr(stream)), "hashprune insert")

    def insert_segments(self, records: torch.Tensor, segments: torch.Tensor, count: int | None = None,
                        stream: torch.cuda.Stream | None = None) -> None:
        """Merge records described by segments (``edges.emit_edge_segments``):
        the first ``count`` rows of ``segments`` (int32 [n, 4]: src, first
        record lo / hi, count) index into ``records`` (int32 [m, 4]).  Same
        result as ``insert`` of the records.  Synchronises the stream."""
        for t in (records, segments):
            if t.dtype != torch.int32 or t.dim() != 2 or t.shape[1] != 4:
                raise ValueError("records and segments must be int32 [n, 4] tensors")
        n = segments.shape[0] if count is None else int(count)
        if n > segments.shape[0]:
            raise ValueError(f"count {n} exceeds the {segments.shape[0]} segments given")
        N.check(self._lib.tessa_hashprune_insert_segments(self._h, _ptr(records), _ptr(segments), n,
                                                          _stream_ptr(stream)), "hashprune insert segments")

    def clear(self, stream: torch.cuda.Stream | None = None) -> None:
        N.check(self._lib.tessa_hashprune_clear(self._h, _stream_ptr(stream)), "hashprune clear")

    def slots(self, stream: torch.cuda.Stream | None = None):
        """(targets int32 [num_points, l_max] (0xFFFFFFFF = unused), hashes int16,
        dists f32, counts int32 [num_points]) in slot order (ascending hash),
        then, with a backfill policy, the row's backups in priority order."""
        t = torch.empty((self.num_points, self.l_max), dtype=torch.int32, device=self.device)
        hs = torch.empty((self.num_points, self.l_max), dtype=torch.int16, device=self.device)
        d = torch.empty((self.num_points, self.l_max), dtype=torch.float32, device=self.device)
        c = torch.empty(self.num_points, dtype=torch.int32, device=self.device)
        N.check(self._lib.tessa_hashprune_neighbors(self._h, _ptr(t), _ptr(hs), _ptr(d), _ptr(c),
                                                    _stream_ptr(stream)), "hashprune neighbors")
        return t, hs, d, c

    def neighbors(self, stream: torch.cuda.Stream | None = None):
        """(targets int32 [num_points, l_max], counts int32 [num_points])."""
        t = torch.empty((self.num_points, self.l_max), dtype=torch.int32, device=self.device)
        c = torch.empty(self.num_points, dtype=torch.int32, device=self.device)
        N.check(self._lib.tessa_hashprune_neighbors(self._h, _ptr(t), None, None, _ptr(c), _stream_ptr(stream)),
                "hashprune neighbors")
        return t, c


def reduce_spill_records_ordered(num_points: int, l_max: int, records, device="cuda",
                                 backfill: HashPruneBackfill | None = None) -> list[list[int]]:
    """reduce_spill_artifacts_ordered (spill_hashprune.rs:875-892) over host or
    device records: each point's neighbour ids in slot order."""
    with HashPruneReducer(num_points, l_max, device, backfill) as hp:
        hp.insert(records)
        t, c = hp.neighbors()
        torch.cuda.synchronize(hp.device)
        tt = t.cpu().numpy().view(np.uint32)
        cc = c.cpu().numpy()
    return [tt[p, :cc[p]].tolist() for p in range(num_points)]
