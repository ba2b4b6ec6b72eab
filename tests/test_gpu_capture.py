"""TESSA capture from a real GPU subtree run: the sampled leaf tasks are the
run's leaves (as global-id sets), the capture round-trips through the
reference's fixture format, and replaying the captured tasks through the
leaf operator matches the oracle bit for bit."""
import numpy as np
import pytest

from gpu_helpers import assert_same, require_gpu, run_leaf, to_dev_sq8
from shear_amd import _native as N
from shear_amd import capture as CP
from shear_amd import datagen
from shear_amd import subtree as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


def test_capture_and_replay_of_subtree_leaves(gpu, orc, tmp_path):
    n, dim = 6000, 64
    x = datagen.gmm_numpy(n, dim, 8, 0.3, 12)
    codes, scales, norms = orc.quantize(x)
    gids = np.random.default_rng(12).permutation(n).astype(np.uint32)
    sess = S.SubtreeSession(0)
    sess.upload(codes, scales, norms, gids, dim)
    out = sess.run(S.GpuSubtreePartitionRequest(point_ids=gids, parent_points=n, min_recurse_size=64),
                   S.PiPNNSubtreeParams(leaf_knn=16, c_max=1024, fanout_second=2, psamp_fraction=0.01, random_seed=5))
    sampler = CP.TessaCaptureSampler(42)
    kept = CP.observe_subtree_leaves(sampler, out, gids, codes.shape[1])
    sel = sampler.finish()
    assert kept > 0 and len(sel.leaf_tasks) == kept
    rows = out.leaf_row_ids[: out.leaf_rows].cpu().numpy().view(np.uint32)
    starts = out.leaf_starts[: out.leaf_count].cpu().numpy()
    sizes = out.leaf_sizes[: out.leaf_count].cpu().numpy()
    leaves = {tuple(sorted(gids[rows[s:s + c]].tolist())) for s, c in zip(starts, sizes)}
    assert all(tuple(t.member_ids) in leaves for t in sel.leaf_tasks)

    ds = {"canonical_base_path": "/data/base.fbin", "rows": n, "dimension": dim, "header_sha256": "ab" * 32}
    prov = {"seed": 42, "git_commit": "local", "binary_sha256": "cd" * 32, "command_sha256": "ef" * 32,
            "root_leader_hash": 1, "d0_partition_hash": 2, "d0_task_list_hash": 3}
    CP.write_tessa_capture(tmp_path, ds, prov, sel)
    _, loaded = CP.load_tessa_capture(tmp_path, ds)
    assert [t.task_hash for t in loaded.leaf_tasks] == sorted(
        (t.task_hash for t in sel.leaf_tasks),
        key=lambda h: next((CP.leaf_size_bin(len(t.member_ids)), t.priority, t.task_hash)
                           for t in sel.leaf_tasks if t.task_hash == h))

    # replay the captured tasks: global ids -> resident rows
    row_of = np.empty(n, np.int64)
    row_of[gids] = np.arange(n)
    members = np.concatenate([row_of[np.asarray(t.member_ids)] for t in loaded.leaf_tasks]).astype(np.uint32)
    counts = np.array([len(t.member_ids) for t in loaded.leaf_tasks])
    offs = np.concatenate([[0], np.cumsum(counts)[:-1]])
    k = loaded.leaf_tasks[0].k
    want_ids, want_d = orc.leaf_topk(codes, scales, norms, gids, members, offs, counts, k)
    ids, d, _ = run_leaf(to_dev_sq8(codes, scales, norms, dim), gids, members, offs, counts, k, N.EXEC_MFMA)
    assert_same(ids, d, want_ids, want_d, "captured leaf tasks")


def _oracle_passes(orc, codes, scales, norms, gids, *, seed, fan, leaf_max, psamp, max_leaders, min_members):
    """The oracle partition's COUNT passes (resident rows mapped to global ids),
    as sorted (depth, attempt, fanout, members, leaders) tuples."""
    from shear_amd import subtree as S

    n = len(gids)
    plan = S.plan_subtree(n, 8, min(max_leaders, 128), fan, None, leaf_max)
    rseed = orc.subtree_root_seed(seed, 0, n, n, 64)
    leaves, ctr, passes = orc.subtree_partition(codes, scales, norms, seed=rseed, max_leaders=min(max_leaders, 128),
                                                fanout_second=fan, leaf_min=plan.leaf_min, leaf_max=plan.leaf_max,
                                                psamp_fraction=psamp, max_leaf_count=plan.max_leaf_count,
                                                max_leaf_rows=plan.max_leaf_rows, trace_min_members=min_members)
    assert leaves is not None, "oracle partition overflowed"
    return sorted((p["depth"], p["attempt"], p["fanout"], tuple(gids[p["members"]].tolist()),
                   tuple(gids[p["leaders"]].tolist())) for p in passes)


def _gpu_passes(tasks):
    return sorted((t["depth"], t["retry"], t["r_h"], tuple(t["member_ids"].tolist()), tuple(t["leader_ids"].tolist()))
                  for t in tasks)


CAPTURE_CASES = [
    # n, dim, comps, sigma, fanout, leaf_max, psamp, max_leaders: the second forces split retries
    (20000, 64, 16, 0.3, 2, 1024, 0.01, 4),
    (8000, 32, 3, 0.05, 2, 512, 0.001, 2),
]


@pytest.mark.parametrize("case", CAPTURE_CASES, ids=["levels", "retries"])
def test_assignment_capture_matches_oracle_passes(gpu, orc, case):
    # every captured task is a COUNT pass the oracle's partition makes on the
    # same rows: same depth, attempt, fanout, member set and order, leaders
    n, dim, comps, sigma, fan, lmax, ps, ml = case
    x = datagen.gmm_numpy(n, dim, comps, sigma, 21)
    codes, scales, norms = orc.quantize(x)
    gids = np.random.default_rng(21).permutation(1 << 20)[:n].astype(np.uint32)
    sess = S.SubtreeSession(0)
    sess.upload(codes, scales, norms, gids, dim)
    sess.set_assignment_capture(256)
    sess.run(S.GpuSubtreePartitionRequest(point_ids=gids, parent_points=n, min_recurse_size=64),
             S.PiPNNSubtreeParams(leaf_knn=8, c_max=lmax, fanout_second=fan, psamp_fraction=ps, max_leaders=ml,
                                  random_seed=9))
    got = _gpu_passes(sess.captured_assignments())
    want = _oracle_passes(orc, codes, scales, norms, gids, seed=9, fan=fan, leaf_max=lmax, psamp=ps,
                          max_leaders=ml, min_members=256)
    assert len(got) == len(want) and got == want, "captured passes differ from the oracle's COUNT passes"
    if ml == 2:
        assert any(p[1] > 0 for p in got), "the retry case made no retry pass"
    # an upload clears the capture (its rows name the replaced set)
    sess.upload(codes, scales, norms, gids, dim)
    assert sess.captured_assignments() == []
    sess.set_assignment_capture(0)


def test_assignment_capture_and_replay(gpu, orc, tmp_path):
    # the partition's assignment passes, captured from the level loop, replayed
    # through the assignment kernel: bit-exact vs the oracle; then sampled and
    # written as capture fixtures
    import torch

    from shear_amd import tessa as T

    n, dim = 20000, 64
    x = datagen.gmm_numpy(n, dim, 16, 0.3, 21)
    codes, scales, norms = orc.quantize(x)
    gids = np.random.default_rng(21).permutation(1 << 20)[:n].astype(np.uint32)
    sess = S.SubtreeSession(0)
    sess.upload(codes, scales, norms, gids, dim)
    sess.set_assignment_capture(256)
    # four leaders per node: the root's children (~10k rows) are large nodes too,
    # so passes at depth 1 go through the level loop as well
    sess.run(S.GpuSubtreePartitionRequest(point_ids=gids, parent_points=n, min_recurse_size=64),
             S.PiPNNSubtreeParams(leaf_knn=8, c_max=1024, fanout_second=2, psamp_fraction=0.01, max_leaders=4,
                                  random_seed=9))
    tasks = sess.captured_assignments()
    assert _gpu_passes(tasks) == _oracle_passes(orc, codes, scales, norms, gids, seed=9, fan=2, leaf_max=1024,
                                                psamp=0.01, max_leaders=4, min_members=256)
    assert tasks and tasks[0]["depth"] == 0 and tasks[0]["retry"] == 0
    assert sorted(tasks[0]["member_ids"].tolist()) == sorted(gids.tolist())  # the root holds every row once
    gset = set(gids.tolist())
    for t in tasks:
        assert len(t["member_ids"]) >= 256 and 1 <= len(t["leader_ids"]) <= 128 and 1 <= t["r_h"] <= 4
        assert t["padded_dim"] == codes.shape[1] and set(t["leader_ids"].tolist()) <= gset
    assert any(t["depth"] > 0 for t in tasks)

    row_of = np.zeros(1 << 20, np.int64)
    row_of[gids] = np.arange(n)
    members, leaders, mo, mc, lo, lc, rh = [], [], [], [], [], [], []
    for t in tasks:
        mo.append(len(members))
        mc.append(len(t["member_ids"]))
        members += row_of[t["member_ids"]].tolist()
        lo.append(len(leaders))
        lc.append(len(t["leader_ids"]))
        leaders += row_of[t["leader_ids"]].tolist()
        rh.append(t["r_h"])
    lay = T.AssignLayouts.from_host(members, leaders, mo, mc, lo, lc, rh)
    ids, d, ctr = T.assignment_replay(to_dev_sq8(codes, scales, norms, dim),
                                      torch.from_numpy(gids.view(np.int32)).to(gpu), lay)
    torch.cuda.synchronize()
    want_ids, want_d = orc.assign_replay(codes, scales, norms, gids, members, leaders, mo, mc, lo, lc, rh)
    assert_same(ids.cpu().numpy().view(np.uint32), d.cpu().numpy(), want_ids, want_d, "captured assignment tasks")

    sampler = CP.TessaCaptureSampler(42)
    kept = CP.observe_captured_assignments(sampler, sess)
    sel = sampler.finish()
    # bins keep their 16 best (priority, hash): later tasks can evict earlier ones
    assert 0 < len(sel.assignment_tasks) <= kept and sum(map(sum, sel.bin_counts.assignment_observed)) == len(tasks)
    ds = {"canonical_base_path": "/data/base.fbin", "rows": 1 << 20, "dimension": dim, "header_sha256": "ab" * 32}
    prov = {"seed": 42, "git_commit": "local", "binary_sha256": "cd" * 32, "command_sha256": "ef" * 32,
            "root_leader_hash": 1, "d0_partition_hash": 2, "d0_task_list_hash": 3}
    CP.write_tessa_capture(tmp_path, ds, prov, sel)
    assert len(CP.load_tessa_capture(tmp_path, ds)[1].assignment_tasks) == len(sel.assignment_tasks)
    sess.set_assignment_capture(0)
