"""The replay command (tessa_operator_replay run) on a capture the build's own
capture writer produced from a GPU subtree run: formal 5 + 20 rotated sweeps,
the exact and MFMA executors identical bit for bit (the replay's own check),
every mode deterministic across measured sweeps, the four output files
written create-new; the exact executor's leaf output checked against the CPU
oracle on the same prepared rows; a second run into the same directory and a
wrong seed refused."""
import json

import numpy as np
import pytest

from gpu_helpers import assert_same, require_gpu
from shear_amd import capture as CP
from shear_amd import datagen
from shear_amd import replay as R
from shear_amd import subtree as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    return require_gpu()


@pytest.fixture(scope="module")
def captured(tmp_path_factory, gpu):
    """(fbin path, capture dir, x): a subtree run's sampled leaf tasks and
    assignment passes written as a capture of a 12,000 x 64 .fbin."""
    from oracle import pyoracle as orc

    d = tmp_path_factory.mktemp("replay")
    n, dim = 12000, 64
    x = datagen.gmm_numpy(n, dim, 8, 0.3, 51)
    base = d / "base.fbin"
    with open(base, "wb") as f:
        f.write(np.array([n, dim], "<u4").tobytes())
        f.write(x.astype("<f4").tobytes())
    codes, scales, norms = orc.quantize(x)
    gids = np.arange(n, dtype=np.uint32)  # global id = base row
    sess = S.SubtreeSession(0)
    sess.upload(codes, scales, norms, gids, dim)
    sess.set_assignment_capture(256)
    out = sess.run(S.GpuSubtreePartitionRequest(point_ids=gids, parent_points=n, min_recurse_size=64),
                   S.PiPNNSubtreeParams(leaf_knn=16, c_max=1024, fanout_second=2, psamp_fraction=0.01,
                                        max_leaders=4, random_seed=5))
    sampler = CP.TessaCaptureSampler(42)
    CP.observe_subtree_leaves(sampler, out, gids, codes.shape[1])
    CP.observe_captured_assignments(sampler, sess)
    sel = sampler.finish()
    assert sel.leaf_tasks and sel.assignment_tasks
    prov = {"seed": 42, "git_commit": "local", "binary_sha256": "cd" * 32, "command_sha256": "ef" * 32,
            "root_leader_hash": 1, "d0_partition_hash": 2, "d0_task_list_hash": 3}
    cap = d / "capture"
    CP.write_tessa_capture(cap, CP.dataset_metadata(base), prov, sel)
    return base, cap, x


def test_formal_replay_run(captured, orc, tmp_path):
    base, cap, x = captured
    cfg = R.TessaReplayRunConfig(seed=42, warmup_sweeps=5, measured_sweeps=20, formal=True,
                                 manifest_path=str(cap / CP.MANIFEST_FILE), base_path=str(base),
                                 output_dir=str(tmp_path / "out"))
    out = R.run_tessa_operator_replay(cfg)
    for f in ("samples.tsv", "task_metrics.tsv", "summary.json", "summary.md"):
        assert (out / f).is_file()
    assert not (out / "failure.json").exists()
    summary = json.loads((out / "summary.json").read_text())
    assert summary["a2_a3_candidate_ids_and_distance_bits_exact"] and summary["formal"]
    modes = {m["mode"]: m for m in summary["modes"]}
    assert set(modes) == {m.value for m in R.RUN_MODES}
    a3 = modes[R.TessaReplayMode.A3_SQ8_WMMA_BATCH8.value]
    assert a3["leaf_overlap_at_k"]["exact_task_fraction"] == 1.0 and a3["assignment_overlap_at_rh"]["macro_mean"] == 1.0
    lines = (out / "samples.tsv").read_text().splitlines()
    # per sweep and mode: assignment + total, plus leaf for the two leaf modes
    assert len(lines) == 1 + 25 * (4 * 2 + 2)
    assert lines[0].split("\t")[:6] == ["phase", "sweep", "order", "mode", "task_kind", "event_ms"]
    assert sum(1 for ln in lines[1:] if ln.startswith("measured")) == 20 * 10

    # the exact executor's leaf result on the prepared rows equals the oracle's
    from shear_amd import capture as CP2

    manifest, sel = CP2.load_tessa_capture(cap, CP2.dataset_metadata(base))
    prep = R.prepare_tessa_replay(manifest, sel, base)
    sess = R.ReplaySession(0, prep)
    a2 = sess.run_mode(R.TessaReplayMode.A2_SQ8_DP4A_BATCH1)
    sess.close()
    codes, scales, norms = orc.quantize(x[prep.global_ids.astype(np.int64)])
    lay = prep.leaf_layouts
    want_ids, want_d = orc.leaf_topk(codes, scales, norms, prep.global_ids, prep.leaf_members,
                                     [t[0] for t in lay], [t[1] for t in lay], prep.leaf_k)
    assert_same(a2.leaf_ids, a2.leaf_dists, want_ids, want_d, "replay A2 leaf vs oracle")

    # create-new outputs: a second run into the same directory is refused
    with pytest.raises(R.ReplayError, match="refusing to overwrite"):
        R.run_tessa_operator_replay(cfg)


def test_replay_seed_and_formal_contract(captured, tmp_path):
    base, cap, _ = captured
    with pytest.raises(R.ReplayError, match="seed mismatch"):
        R.run_tessa_operator_replay(R.TessaReplayRunConfig(seed=43, warmup_sweeps=1, measured_sweeps=1, formal=False,
                                                           manifest_path=str(cap), base_path=str(base),
                                                           output_dir=str(tmp_path / "o1")))
    with pytest.raises(ValueError, match="formal replay requires exactly 5 warmup and 20 measured"):
        R.run_tessa_operator_replay(R.TessaReplayRunConfig(seed=42, warmup_sweeps=1, measured_sweeps=2, formal=True,
                                                           manifest_path=str(cap), base_path=str(base),
                                                           output_dir=str(tmp_path / "o2")))
