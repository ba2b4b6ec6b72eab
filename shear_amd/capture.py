"""TESSA capture writer: sampled leaf and assignment tasks of real builds,
written as replay fixtures in the reference's format.

Host mirror of shear-core/src/algorithm/pipnn/tessa_capture.rs and the
finalize step of tessa_replay.rs:240-318:

* task hashes and priorities   StableFnv1a64 over a domain string and the fields'
                               little-endian bytes; membership digest (count,
                               wrapping sum and rotated xor of the SplitMix64
                               finaliser of each id) :177-300
* bins                         :206-231 (assignment rows 256..1024 / ..8192 / more,
                               leaders 1..16 / ..32 / ..64 / ..128; leaves 256..512 /
                               ..896 / ..1280)
* ``TessaCaptureSampler``      bottom-k by (priority, hash) per bin, 16 assignment /
                               64 leaf tasks kept, duplicates by hash ignored :350-458
* fragments                    ``fragment-{request_hash:016x}.json``, merge :460-597
* ``write_tessa_capture``      manifest.json + three u32le member/leader files :599-690
* ``load_tessa_capture``       with the reference's checks :692-1050
* ``finalize_tessa_capture``   tessa_replay.rs:240-318

The reference samples inside its persistent kernel (compute_backend.rs:
5415-5546); here the leaf layout of a subtree run is already in HBM, so
``observe_subtree_leaves`` samples it from the host after the run.
Assignment tasks come from the partition's level loop
(``SubtreeSession.set_assignment_capture``, ``observe_captured_assignments``).
"""
from __future__ import annotations

import hashlib
import json
import os
import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

VERSION = 1
MANIFEST_FILE = "manifest.json"
ASSIGNMENT_MEMBERS_FILE = "assignment_members.u32le"
ASSIGNMENT_LEADERS_FILE = "assignment_leaders.u32le"
LEAF_MEMBERS_FILE = "leaf_members.u32le"
ASSIGNMENT_ROW_BINS, ASSIGNMENT_LEADER_BINS, LEAF_SIZE_BINS = 3, 4, 3
ASSIGNMENT_BIN_LIMIT, LEAF_BIN_LIMIT = 16, 64
_M64 = (1 << 64) - 1


class CaptureError(RuntimeError):
    pass


class _Fnv:
    def __init__(self, domain: bytes):
        self.h = 0xCBF29CE484222325
        self.write(domain)

    def write(self, data: bytes):
        h = self.h
        for b in data:
            h = ((h ^ b) * 0x100000001B3) & _M64
        self.h = h

    def u32(self, v):
        self.write(struct.pack("<I", v & 0xFFFFFFFF))

    def u64(self, v):
        self.write(struct.pack("<Q", v & _M64))

    def finish(self) -> int:
        return self.h or 1


def mix_membership_id(value: int) -> int:
    z = (value + 0x9E3779B97F4A7C15) & _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def membership_digest(ids) -> tuple[int, int]:
    s = x = 0
    for i in ids:
        m = mix_membership_id(int(i))
        r = int(i) & 63
        s = (s + m) & _M64
        x ^= ((m << r) | (m >> (64 - r))) & _M64 if r else m
    return s, x


def _digest(h: _Fnv, ids):
    s, x = membership_digest(ids)
    h.u64(len(ids))
    h.u64(s)
    h.u64(x)


def priority_for_task(seed: int, task_hash: int) -> int:
    h = _Fnv(b"SHEAR-TESSA-PRIORITY\0")
    h.u64(seed)
    h.u64(task_hash)
    return h.finish()


def assignment_task_hash(seed, depth, retry, r_h, padded_dim, member_ids, leader_ids) -> int:
    h = _Fnv(b"SHEAR-TESSA-ASSIGNMENT\0")
    h.u64(seed)
    for v in (depth, retry, r_h, padded_dim):
        h.u32(v)
    _digest(h, member_ids)
    h.u64(len(leader_ids))
    for v in leader_ids:
        h.u32(int(v))
    return h.finish()


def leaf_task_hash(seed, k, padded_dim, member_ids) -> int:
    h = _Fnv(b"SHEAR-TESSA-LEAF\0")
    h.u64(seed)
    h.u32(k)
    h.u32(padded_dim)
    _digest(h, member_ids)
    return h.finish()


def tessa_request_hash(seed: int, member_ids) -> int:
    h = _Fnv(b"SHEAR-TESSA-REQUEST\0")
    h.u64(seed)
    _digest(h, member_ids)
    return h.finish()


def assignment_row_bin(rows: int):
    return 0 if 256 <= rows <= 1024 else 1 if 1025 <= rows <= 8192 else 2 if rows >= 8193 else None


def assignment_leader_bin(leaders: int):
    for b, hi in enumerate((16, 32, 64, 128)):
        if 1 <= leaders <= hi:
            return b
    return None


def leaf_size_bin(rows: int):
    return 0 if 256 <= rows <= 512 else 1 if 513 <= rows <= 896 else 2 if 897 <= rows <= 1280 else None


@dataclass
class AssignmentTask:
    task_hash: int
    priority: int
    depth: int
    retry: int
    r_h: int
    padded_dim: int
    member_ids: list
    leader_ids: list


@dataclass
class LeafTask:
    task_hash: int
    priority: int
    k: int
    padded_dim: int
    member_ids: list


def make_assignment_task(seed, depth, retry, r_h, padded_dim, member_ids, leader_ids) -> AssignmentTask:
    m = sorted(int(i) for i in member_ids)
    lids = [int(i) for i in leader_ids]
    th = assignment_task_hash(seed, depth, retry, r_h, padded_dim, m, lids)
    return AssignmentTask(th, priority_for_task(seed, th), depth, retry, r_h, padded_dim, m, lids)


def make_leaf_task(seed, k, padded_dim, member_ids) -> LeafTask:
    m = sorted(int(i) for i in member_ids)
    th = leaf_task_hash(seed, k, padded_dim, m)
    return LeafTask(th, priority_for_task(seed, th), k, padded_dim, m)


def _zeros2():
    return [[0] * ASSIGNMENT_LEADER_BINS for _ in range(ASSIGNMENT_ROW_BINS)]


@dataclass
class BinCounts:
    assignment_observed: list = field(default_factory=_zeros2)
    assignment_selected: list = field(default_factory=_zeros2)
    leaf_observed: list = field(default_factory=lambda: [0] * LEAF_SIZE_BINS)
    leaf_selected: list = field(default_factory=lambda: [0] * LEAF_SIZE_BINS)


@dataclass
class Selection:
    assignment_tasks: list
    leaf_tasks: list
    bin_counts: BinCounts


class TessaCaptureSampler:
    """Bottom-k sampler per bin (tessa_capture.rs:350-458)."""

    def __init__(self, seed: int):
        self.seed = seed
        self.assignment_bins = [[[] for _ in range(ASSIGNMENT_LEADER_BINS)] for _ in range(ASSIGNMENT_ROW_BINS)]
        self.leaf_bins = [[] for _ in range(LEAF_SIZE_BINS)]
        self.counts = BinCounts()

    @staticmethod
    def _keep(bin_, task, limit, what):
        for e in bin_:
            if e.task_hash == task.task_hash:
                if e != task:
                    raise CaptureError(f"{what} task hash collision for {task.task_hash}")
                return False
        bin_.append(task)
        bin_.sort(key=lambda t: (t.priority, t.task_hash))
        if len(bin_) > limit:
            bin_.pop()
        return True

    def observe_assignment(self, task: AssignmentTask) -> bool:
        t = make_assignment_task(self.seed, task.depth, task.retry, task.r_h, task.padded_dim, task.member_ids,
                                 task.leader_ids)
        rb, lb = assignment_row_bin(len(t.member_ids)), assignment_leader_bin(len(t.leader_ids))
        if rb is None or lb is None:
            return False
        self.counts.assignment_observed[rb][lb] += 1
        return self._keep(self.assignment_bins[rb][lb], t, ASSIGNMENT_BIN_LIMIT, "assignment")

    def observe_leaf(self, task: LeafTask) -> bool:
        t = make_leaf_task(self.seed, task.k, task.padded_dim, task.member_ids)
        sb = leaf_size_bin(len(t.member_ids))
        if sb is None:
            return False
        self.counts.leaf_observed[sb] += 1
        return self._keep(self.leaf_bins[sb], t, LEAF_BIN_LIMIT, "leaf")

    def finish(self) -> Selection:
        a, l = [], []
        for rb in range(ASSIGNMENT_ROW_BINS):
            for lb in range(ASSIGNMENT_LEADER_BINS):
                b = sorted(self.assignment_bins[rb][lb], key=lambda t: (t.priority, t.task_hash))
                self.counts.assignment_selected[rb][lb] = len(b)
                a += b
        for sb in range(LEAF_SIZE_BINS):
            b = sorted(self.leaf_bins[sb], key=lambda t: (t.priority, t.task_hash))
            self.counts.leaf_selected[sb] = len(b)
            l += b
        return Selection(a, l, self.counts)


def observe_subtree_leaves(sampler: TessaCaptureSampler, out, global_ids, padded_dim: int) -> int:
    """Observe every leaf of a subtree run's device output (leaf layout,
    resident row -> global id map): the leaf tasks the reference's kernel
    samples (compute_backend.rs:5415-5546).  Returns the number kept."""
    lc, lr = out.leaf_count, out.leaf_rows
    rows = out.leaf_row_ids[:lr].cpu().numpy().view(np.uint32)
    starts = out.leaf_starts[:lc].cpu().numpy()
    sizes = out.leaf_sizes[:lc].cpu().numpy()
    g = np.asarray(global_ids.cpu().numpy() if hasattr(global_ids, "cpu") else global_ids).view(np.uint32)
    kept = 0
    for s, n in zip(starts.tolist(), sizes.tolist()):
        if leaf_size_bin(n) is None:
            continue
        k = min(out.k, n - 1)
        kept += sampler.observe_leaf(LeafTask(0, 0, k, padded_dim, g[rows[s:s + n]].tolist()))
    return kept


def observe_captured_assignments(sampler: TessaCaptureSampler, session) -> int:
    """Observe the assignment passes a SubtreeSession recorded in its last run
    (``set_assignment_capture``).  Returns the number kept."""
    kept = 0
    for t in session.captured_assignments():
        kept += sampler.observe_assignment(AssignmentTask(0, 0, t["depth"], t["retry"], t["r_h"], t["padded_dim"],
                                                          t["member_ids"].tolist(), t["leader_ids"].tolist()))
    return kept


# ---- serialization (serde_json pretty layout: two-space indent, field order) ----

def _task_dict(t):
    return dict(t.__dict__)


def _counts_dict(c: BinCounts):
    return {"assignment_observed": c.assignment_observed, "assignment_selected": c.assignment_selected,
            "leaf_observed": c.leaf_observed, "leaf_selected": c.leaf_selected}


def _selection_dict(s: Selection):
    return {"assignment_tasks": [_task_dict(t) for t in s.assignment_tasks],
            "leaf_tasks": [_task_dict(t) for t in s.leaf_tasks], "bin_counts": _counts_dict(s.bin_counts)}


def _selection_from(d) -> Selection:
    c = d["bin_counts"]
    return Selection([AssignmentTask(**t) for t in d["assignment_tasks"]], [LeafTask(**t) for t in d["leaf_tasks"]],
                     BinCounts(c["assignment_observed"], c["assignment_selected"], c["leaf_observed"],
                               c["leaf_selected"]))


def _json_bytes(obj) -> bytes:
    return (json.dumps(obj, indent=2) + "\n").encode()


def write_tessa_capture_fragment(dir_, request_hash: int, selection: Selection) -> Path:
    d = Path(dir_)
    d.mkdir(parents=True, exist_ok=True)
    data = _json_bytes({"version": VERSION, "request_hash": request_hash, "selection": _selection_dict(selection)})
    path = d / f"fragment-{request_hash:016x}.json"
    try:
        fd = os.open(path, os.O_WRONLY | os.O_CREAT | os.O_EXCL, 0o644)
    except FileExistsError:
        if path.read_bytes() != data:
            raise CaptureError(f"existing TESSA fragment {path} differs from request {request_hash:016x}")
        return path
    with os.fdopen(fd, "wb") as f:
        f.write(data)
        f.flush()
        os.fsync(f.fileno())
    return path


def merge_tessa_capture_fragments(dir_, seed: int) -> Selection:
    paths = sorted(p for p in Path(dir_).iterdir() if p.name.startswith("fragment-") and p.name.endswith(".json"))
    if not paths:
        raise CaptureError(f"no TESSA capture fragments found in {dir_}")
    sampler = TessaCaptureSampler(seed)
    observed = BinCounts()
    seen = set()
    for p in paths:
        frag = json.loads(p.read_bytes())
        if frag["version"] != VERSION:
            raise CaptureError(f"unsupported TESSA fragment version {frag['version']} in {p}")
        if frag["request_hash"] in seen:
            raise CaptureError(f"duplicate TESSA request hash {frag['request_hash']:016x}")
        seen.add(frag["request_hash"])
        sel = _selection_from(frag["selection"])
        for rb in range(ASSIGNMENT_ROW_BINS):
            for lb in range(ASSIGNMENT_LEADER_BINS):
                observed.assignment_observed[rb][lb] += sel.bin_counts.assignment_observed[rb][lb]
        for sb in range(LEAF_SIZE_BINS):
            observed.leaf_observed[sb] += sel.bin_counts.leaf_observed[sb]
        for t in sel.assignment_tasks:
            sampler.observe_assignment(t)
        for t in sel.leaf_tasks:
            sampler.observe_leaf(t)
    out = sampler.finish()
    out.bin_counts.assignment_observed = observed.assignment_observed
    out.bin_counts.leaf_observed = observed.leaf_observed
    return out


def _is_sha256(v: str) -> bool:
    return len(v) == 64 and all(c in "0123456789abcdefABCDEF" for c in v)


def dataset_metadata(fbin_path) -> dict:
    """tessa_capture_dataset_metadata (tessa_capture.rs:52-86): canonical path,
    rows and dimension from the .fbin header, SHA-256 of its 8 header bytes."""
    p = Path(fbin_path).resolve()
    head = p.read_bytes()[:8] if p.stat().st_size < (1 << 20) else open(p, "rb").read(8)
    if len(head) < 8:
        raise CaptureError(f"failed to read capture dataset header {p}")
    rows, dim = struct.unpack("<ii", head)
    meta = {"canonical_base_path": str(p), "rows": rows, "dimension": dim,
            "header_sha256": hashlib.sha256(head).hexdigest()}
    _validate_dataset(meta)
    return meta


def _validate_dataset(d: dict):
    if not d["canonical_base_path"] or not os.path.isabs(d["canonical_base_path"]) or d["rows"] == 0 \
            or d["dimension"] == 0 or not _is_sha256(d["header_sha256"]):
        raise CaptureError(f"invalid capture dataset metadata: path='{d['canonical_base_path']}' rows={d['rows']} "
                           f"dim={d['dimension']} header_sha256='{d['header_sha256']}'")


def _validate_provenance(p: dict):
    if not p["git_commit"] or not _is_sha256(p["binary_sha256"]) or not _is_sha256(p["command_sha256"]) \
            or p["root_leader_hash"] == 0 or p["d0_partition_hash"] == 0 or p["d0_task_list_hash"] == 0:
        raise CaptureError("invalid TESSA capture provenance")


def _validate_selection(s: Selection, seed: int, rows: int):
    hashes = set()
    sel_a = _zeros2()
    for t in s.assignment_tasks:
        rb, lb = assignment_row_bin(len(t.member_ids)), assignment_leader_bin(len(t.leader_ids))
        if rb is None:
            raise CaptureError("assignment task is outside configured row bins")
        if lb is None:
            raise CaptureError("assignment task is outside configured leader bins")
        sel_a[rb][lb] += 1
        if sel_a[rb][lb] > ASSIGNMENT_BIN_LIMIT:
            raise CaptureError(f"assignment capture bin ({rb}, {lb}) exceeds limit {ASSIGNMENT_BIN_LIMIT}")
        _validate_ids(t.member_ids, rows, "assignment member", sorted_label="assignment members")
        _validate_ids(t.leader_ids, rows, "assignment leader")
        if t.r_h == 0 or t.r_h > len(t.leader_ids):
            raise CaptureError(f"assignment task {t.task_hash} has invalid r_h {t.r_h} for {len(t.leader_ids)} leaders")
        if t.padded_dim == 0:
            raise CaptureError(f"assignment task {t.task_hash} has zero padded_dim")
        want = assignment_task_hash(seed, t.depth, t.retry, t.r_h, t.padded_dim, t.member_ids, t.leader_ids)
        _check_hash(t, want, seed, hashes)
    sel_l = [0] * LEAF_SIZE_BINS
    for t in s.leaf_tasks:
        sb = leaf_size_bin(len(t.member_ids))
        if sb is None:
            raise CaptureError("leaf task is outside configured size bins")
        sel_l[sb] += 1
        if sel_l[sb] > LEAF_BIN_LIMIT:
            raise CaptureError(f"leaf capture bin {sb} exceeds limit {LEAF_BIN_LIMIT}")
        _validate_ids(t.member_ids, rows, "leaf member", sorted_label="leaf members")
        if t.k == 0 or t.k >= len(t.member_ids) or t.padded_dim == 0:
            raise CaptureError(f"leaf task {t.task_hash} has invalid k {t.k} or padded_dim {t.padded_dim} "
                               f"for {len(t.member_ids)} members")
        _check_hash(t, leaf_task_hash(seed, t.k, t.padded_dim, t.member_ids), seed, hashes)
    c = s.bin_counts
    if c.assignment_selected != sel_a or c.leaf_selected != sel_l:
        raise CaptureError("capture selected bin counts do not match task records")
    if any(c.assignment_observed[r][b] < sel_a[r][b] for r in range(ASSIGNMENT_ROW_BINS)
           for b in range(ASSIGNMENT_LEADER_BINS)):
        raise CaptureError("capture assignment observed count is smaller than selected count")
    if any(o < q for o, q in zip(c.leaf_observed, sel_l)):
        raise CaptureError("capture leaf observed count is smaller than selected count")


def _validate_ids(ids, rows, label, sorted_label=None):
    if sorted_label and any(a > b for a, b in zip(ids, ids[1:])):
        raise CaptureError(f"{sorted_label} are not in canonical sorted order")
    bad = next((i for i in ids if i >= rows), None)
    if bad is not None:
        raise CaptureError(f"{label} id {bad} is outside dataset rows {rows}")


def _check_hash(t, want, seed, hashes):
    if t.task_hash != want or t.priority != priority_for_task(seed, want):
        raise CaptureError(f"TESSA task hash or priority mismatch for task {t.task_hash}")
    if t.task_hash in hashes:
        raise CaptureError(f"duplicate TESSA task hash {t.task_hash}")
    hashes.add(t.task_hash)


def write_tessa_capture(dir_, dataset: dict, provenance: dict, selection: Selection) -> Path:
    _validate_dataset(dataset)
    _validate_provenance(provenance)
    s = Selection(sorted(selection.assignment_tasks, key=lambda t: (
        assignment_row_bin(len(t.member_ids)) or 0, assignment_leader_bin(len(t.leader_ids)) or 0, t.priority,
        t.task_hash)), sorted(selection.leaf_tasks, key=lambda t: (leaf_size_bin(len(t.member_ids)) or 0, t.priority,
                                                                     t.task_hash)), selection.bin_counts)
    _validate_selection(s, provenance["seed"], dataset["rows"])
    d = Path(dir_)
    d.mkdir(parents=True, exist_ok=True)
    am, al, lm, ameta, lmeta = [], [], [], [], []
    for t in s.assignment_tasks:
        ameta.append({"task_hash": t.task_hash, "priority": t.priority, "depth": t.depth, "retry": t.retry,
                      "r_h": t.r_h, "padded_dim": t.padded_dim, "member_offset": len(am),
                      "member_len": len(t.member_ids), "leader_offset": len(al), "leader_len": len(t.leader_ids)})
        am += t.member_ids
        al += t.leader_ids
    for t in s.leaf_tasks:
        lmeta.append({"task_hash": t.task_hash, "priority": t.priority, "k": t.k, "padded_dim": t.padded_dim,
                      "member_offset": len(lm), "member_len": len(t.member_ids)})
        lm += t.member_ids
    files = {"assignment_members": ASSIGNMENT_MEMBERS_FILE, "assignment_leaders": ASSIGNMENT_LEADERS_FILE,
             "leaf_members": LEAF_MEMBERS_FILE}
    for name, vals in ((ASSIGNMENT_MEMBERS_FILE, am), (ASSIGNMENT_LEADERS_FILE, al), (LEAF_MEMBERS_FILE, lm)):
        (d / name).write_bytes(np.asarray(vals, "<u4").tobytes())
    manifest = {"version": VERSION, "dataset": dataset, "provenance": provenance,
                "bin_counts": _counts_dict(s.bin_counts), "files": files, "assignment_tasks": ameta,
                "leaf_tasks": lmeta}
    path = d / MANIFEST_FILE
    path.write_bytes(_json_bytes(manifest))
    return path


def load_tessa_capture(dir_, expected_dataset: dict | None = None):
    """(manifest dict, Selection) with the reference's checks."""
    d = Path(dir_)
    m = json.loads((d / MANIFEST_FILE).read_bytes())
    if m["version"] != VERSION:
        raise CaptureError(f"unsupported TESSA capture version {m['version']}")
    _validate_dataset(m["dataset"])
    _validate_provenance(m["provenance"])
    if expected_dataset is not None:
        _validate_dataset(expected_dataset)
        a, e = m["dataset"], expected_dataset
        if (a["rows"], a["dimension"], a["header_sha256"]) != (e["rows"], e["dimension"], e["header_sha256"]):
            raise CaptureError(f"capture dataset identity mismatch: captured rows={a['rows']} dim={a['dimension']} "
                               f"header_sha256={a['header_sha256']}, expected rows={e['rows']} "
                               f"dim={e['dimension']} header_sha256={e['header_sha256']}")
    for name in m["files"].values():
        if os.sep in name or name in ("", ".", ".."):
            raise CaptureError(f"capture file name must be one relative path component: {name}")
    arr = {k: np.fromfile(d / v, "<u4").tolist() for k, v in m["files"].items()}

    def take(vals, off, n, nxt, label):
        if off != nxt:
            raise CaptureError(f"{label} metadata is not contiguous: expected offset {nxt}, got {off}")
        if off + n > len(vals):
            raise CaptureError(f"{label} slice is outside its file")
        return vals[off:off + n], off + n

    na = nl = nm = 0
    at, lt = [], []
    for t in m["assignment_tasks"]:
        mem, na = take(arr["assignment_members"], t["member_offset"], t["member_len"], na, "assignment members")
        lead, nl = take(arr["assignment_leaders"], t["leader_offset"], t["leader_len"], nl, "assignment leaders")
        at.append(AssignmentTask(t["task_hash"], t["priority"], t["depth"], t["retry"], t["r_h"], t["padded_dim"],
                                 mem, lead))
    for t in m["leaf_tasks"]:
        mem, nm = take(arr["leaf_members"], t["member_offset"], t["member_len"], nm, "leaf members")
        lt.append(LeafTask(t["task_hash"], t["priority"], t["k"], t["padded_dim"], mem))
    if (na, nl, nm) != (len(arr["assignment_members"]), len(arr["assignment_leaders"]), len(arr["leaf_members"])):
        raise CaptureError("capture files hold ids no task references")
    c = m["bin_counts"]
    sel = Selection(at, lt, BinCounts(c["assignment_observed"], c["assignment_selected"], c["leaf_observed"],
                                      c["leaf_selected"]))
    _validate_selection(sel, m["provenance"]["seed"], m["dataset"]["rows"])
    return m, sel


def finalize_tessa_capture(fragment_dir, capture_profile_path, provenance_path, output_dir, seed: int) -> Path:
    """tessa_replay.rs:240-318: provenance file {dataset, provenance}, the
    build profile's three hashes checked against it, fragments merged."""
    meta = json.loads(Path(provenance_path).read_bytes())
    prov = meta["provenance"]
    if prov["seed"] != seed:
        raise CaptureError(f"capture seed mismatch: requested={seed} provenance={prov['seed']}")
    profile = json.loads(Path(capture_profile_path).read_bytes())
    for label, path in (("root_leader_hash", ("root_fanout", "root_leader_hash")),
                        ("d0_partition_hash", ("gpu_subtree", "d0_partition_hash")),
                        ("d0_task_list_hash", ("gpu_subtree", "d0_task_list_hash"))):
        v = profile
        for k in path:
            v = v.get(k) if isinstance(v, dict) else None
        if not isinstance(v, int):
            raise CaptureError(f"capture profile is missing numeric {label} at {'.'.join(path)}")
        if v != prov[label]:
            raise CaptureError(f"capture profile {label} mismatch: profile={v} provenance={prov[label]}")
    return write_tessa_capture(output_dir, meta["dataset"], prov, merge_tessa_capture_fragments(fragment_dir, seed))
