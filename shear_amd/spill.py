"""TierLift spill artifacts: edge records written as the reference's spill
part files and segment manifest, and read back.

Host mirror of SpillEdgeSink's on-disk output (paths relative to
shear-core/src/algorithm/pipnn/spill_hashprune.rs):

* record bytes      SpillRecord16 little-endian: src u32, dst u32, hash u16,
                    flags u16, dist f32 (:139-145, CandidateRunWriter::push :231-238)
* shards            src // shard_points, 1,000,000 points by default (:26, :587-596)
* segments          a shard's buffered records sorted by src, written as one
                    segment when the buffer reaches the flush threshold (64 MiB of
                    pending edges, at most 1,000,000 records: :25, :500-505,
                    :616-650, :727-758)
* part files        ``{stem}_shard{shard:05}_part{part:03}.log`` next to the base
                    path, rolled over past 4 GiB (:27, :770-830)
* manifest          ``candidate_segments.manifest``, one CSV line per segment:
                    shard, file, byte offset, byte length, records, src min, src
                    max, sorted flag, ordered by (shard, file, offset) (:28, :536-549, :832-851)

The build keeps records in HBM and merges them on the GPU
(``hashprune.HashPruneReducer``); these files are for interchange with a
host reducer, the reference's included.
"""
from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .edges import EDGE_RECORD_DTYPE

MANIFEST_NAME = "candidate_segments.manifest"
DEFAULT_SHARD_POINTS = 1_000_000
DEFAULT_PART_MAX_BYTES = 4 * 1024 ** 3
DEFAULT_SEGMENT_RECORDS = 1_000_000
RECORD_BYTES = 16


class SpillError(ValueError):
    pass


@dataclass(frozen=True)
class Segment:
    shard_id: int
    file_id: int
    byte_offset: int
    byte_len: int
    record_count: int
    src_min: int
    src_max: int
    sorted_by_src: bool


def part_path(base_path, part_index: int, shard_id: int) -> Path:
    b = Path(base_path)
    stem = b.stem or "candidate"
    return b.parent / f"{stem}_shard{shard_id:05d}_part{part_index:03d}.log"


def _host_records(records, count=None) -> np.ndarray:
    if hasattr(records, "cpu"):  # a device int32 [n, 4] tensor as emitted
        n = records.shape[0] if count is None else int(count)
        return records[:n].contiguous().cpu().numpy().view(np.uint8).reshape(-1).view(EDGE_RECORD_DTYPE)
    r = np.ascontiguousarray(records, EDGE_RECORD_DTYPE)
    return r if count is None else r[: int(count)]


def write_spill_artifacts(base_path, records, count=None, shard_points: int = DEFAULT_SHARD_POINTS,
                          segment_records: int = DEFAULT_SEGMENT_RECORDS,
                          part_max_bytes: int = DEFAULT_PART_MAX_BYTES) -> tuple[list[Path], list[Segment], Path]:
    """Write records (host EDGE_RECORD_DTYPE or device int32 [n, 4]) in arrival
    order as the sink would: per shard, consecutive runs of segment_records
    records sorted by src.  Returns (part files, segments, manifest path)."""
    rec = _host_records(records, count)
    base = Path(base_path)
    base.parent.mkdir(parents=True, exist_ok=True)
    shard_of = rec["src"].astype(np.int64) // shard_points
    parts: dict[tuple[int, int], Path] = {}
    segments: list[Segment] = []
    for shard in np.unique(shard_of).tolist():
        idx = np.nonzero(shard_of == shard)[0]  # arrival order within the shard
        file_id, file_len, fh = 0, 0, None
        for s0 in range(0, len(idx), segment_records):
            seg = rec[idx[s0:s0 + segment_records]]
            seg = seg[np.argsort(seg["src"], kind="stable")]
            nbytes = len(seg) * RECORD_BYTES
            if fh is None or file_len + nbytes > part_max_bytes:
                if fh is not None:
                    fh.close()
                    file_id += 1
                path = part_path(base, file_id, shard)
                parts[(shard, file_id)] = path
                fh, file_len = open(path, "wb"), 0
            fh.write(seg.tobytes())
            segments.append(Segment(shard, file_id, file_len, nbytes, len(seg), int(seg["src"][0]),
                                    int(seg["src"][-1]), True))
            file_len += nbytes
        if fh is not None:
            fh.close()
    segments.sort(key=lambda s: (s.shard_id, s.file_id, s.byte_offset))
    manifest = base.parent / MANIFEST_NAME
    manifest.write_text("".join(f"{s.shard_id},{s.file_id},{s.byte_offset},{s.byte_len},{s.record_count},"
                                f"{s.src_min},{s.src_max},{int(s.sorted_by_src)}\n" for s in segments))
    return [parts[k] for k in sorted(parts)], segments, manifest


def read_segments(manifest_path) -> list[Segment]:
    out = []
    for i, line in enumerate(Path(manifest_path).read_text().splitlines()):
        f = line.split(",")
        if len(f) != 8:
            raise SpillError(f"segment manifest line {i + 1}: expected 8 fields, got {len(f)}")
        v = [int(x) for x in f]
        out.append(Segment(v[0], v[1], v[2], v[3], v[4], v[5], v[6], bool(v[7])))
    return out


def read_spill_artifacts(base_path, shard_points: int = DEFAULT_SHARD_POINTS) -> np.ndarray:
    """All records of the artifacts next to base_path, segment by segment in
    manifest order, with the segment descriptors checked against the bytes."""
    base = Path(base_path)
    segs = read_segments(base.parent / MANIFEST_NAME)
    chunks = []
    for s in segs:
        if s.byte_len != s.record_count * RECORD_BYTES:
            raise SpillError(f"segment of {s.record_count} records has {s.byte_len} bytes")
        with open(part_path(base, s.file_id, s.shard_id), "rb") as fh:
            fh.seek(s.byte_offset)
            data = fh.read(s.byte_len)
        if len(data) != s.byte_len:
            raise SpillError(f"shard {s.shard_id} part {s.file_id}: segment past the end of the file")
        r = np.frombuffer(data, EDGE_RECORD_DTYPE)
        src = r["src"]
        if len(r) and (src.min() != s.src_min or src.max() != s.src_max or np.any(src // shard_points != s.shard_id)):
            raise SpillError(f"shard {s.shard_id} part {s.file_id} offset {s.byte_offset}: sources do not match")
        if s.sorted_by_src and np.any(src[1:] < src[:-1]):
            raise SpillError(f"shard {s.shard_id} part {s.file_id} offset {s.byte_offset}: not sorted by src")
        chunks.append(r)
    return np.concatenate(chunks) if chunks else np.zeros(0, EDGE_RECORD_DTYPE)
