"""The first-tile visit rule of the partition's COUNT kernel, checked on the CPU.

COUNT inserts a row's leader distances into its F slots in leader order with
the reference's comparator (compute_backend.rs:6541-6568: distances within the
tie band 2e-5 compare by a hash key, others by value; insertion :6524-6580),
which is not transitive.  The slots are empty as a row's first 32-leader tile
starts, and the kernel visits only the leaders at or below T, the row's F-th
smallest distance in the tile, unless some distance d > T has
fl(d - T) <= 2e-5 (or a NaN, or fewer than F finite distances), in which case
it visits every leader.  This test restates that rule and the full in-order
insertion in f32 and checks that they leave the same slots on random tiles
built to put many distances inside and just outside the band.  The GPU tests
compare the kernel's leaves with the oracle (which always visits every leader).
"""
import numpy as np

F32 = np.float32
EPS = F32(2e-5)
EMPTY_D = F32(np.finfo(np.float32).max)
EMPTY_L = 0xFFFFFFFF


def _key(point, leader):
    # any deterministic key: the rule must hold for every tie order
    x = (point * 0x9E3779B1 ^ leader * 0x85EBCA77) & 0xFFFFFFFF
    x ^= x >> 15
    return (x * 0x2C1B3C6D) & 0xFFFFFFFF


def _before(d, point, leader, od, oleader):
    if abs(F32(d - od)) <= EPS:
        ck, ok = _key(point, leader), _key(point, oleader)
        return ck < ok or (ck == ok and leader < oleader)
    return bool(d < od)


def _insert(F, bd, bl, d, point, leader):
    if not _before(d, point, leader, bd[F - 1], bl[F - 1]):
        return
    pos = F - 1
    for q in range(F - 1, 0, -1):
        if pos == q and _before(d, point, leader, bd[q - 1], bl[q - 1]):
            bd[q], bl[q] = bd[q - 1], bl[q - 1]
            pos = q - 1
    bd[pos], bl[pos] = d, leader


def _slots(F, dists, point, visit):
    bd, bl = [EMPTY_D] * F, [EMPTY_L] * F
    for q, d in enumerate(dists):
        if visit[q]:
            _insert(F, bd, bl, d, point, q)
    return bd, bl


def _first_tile_visits(F, dists):
    """The kernel's rule: the leaders to visit, or every leader (None)."""
    finite = sorted(float(d) for d in dists if np.isfinite(d))
    if len(finite) < F:
        return None
    T = F32(finite[F - 1])
    near = []
    for d in dists:
        if d <= T:
            near.append(True)
        elif not (F32(d - T) > EPS):  # inside the band above T, or NaN
            return None
        else:
            near.append(False)
    return near


def test_first_tile_rule_leaves_the_same_slots():
    rng = np.random.default_rng(2024)
    taken = fallback = 0
    for case in range(6000):
        F = int(rng.integers(1, 5))
        n = int(rng.choice([32, 32, 20, 5, 3]))
        base = F32(rng.uniform(0.0, 2.0))
        step = F32(rng.choice([1e-6, 1e-5, 1.9e-5, 2.1e-5, 3e-5, 1e-3]))
        d = (base + rng.integers(0, 6, n).astype(F32) * step).astype(F32)
        if case % 50 == 0:
            d[rng.integers(0, n)] = F32(np.inf)  # a row of overflowed norm
        if case % 97 == 0:
            d[rng.integers(0, n)] = F32(0.0)
        point = int(rng.integers(0, 1 << 20))
        full = _slots(F, d, point, [not (F32(x - EMPTY_D) > EPS) for x in d])  # the kernel's visit test, empty slots
        near = _first_tile_visits(F, d)
        if near is None:
            fallback += 1
            continue
        taken += 1
        assert _slots(F, d, point, near) == full, (F, d.tolist(), point)
    # both branches of the rule are exercised
    assert taken > 1000 and fallback > 1000, (taken, fallback)


def test_rule_rejects_a_dropped_band_check():
    """Without the band check the skipped leaders can change the slots: the
    check is what makes the rule exact."""
    rng = np.random.default_rng(7)
    differ = 0
    for _ in range(3000):
        F = int(rng.integers(1, 5))
        d = (F32(1.0) + rng.integers(0, 4, 32).astype(F32) * F32(1e-5)).astype(F32)
        point = int(rng.integers(0, 1 << 20))
        T = F32(sorted(d)[F - 1])
        near = [bool(x <= T) for x in d]
        if _slots(F, d, point, near) != _slots(F, d, point, [True] * 32):
            differ += 1
    assert differ > 0
