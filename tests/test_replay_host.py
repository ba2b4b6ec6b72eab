"""Replay host logic against the reference's own KATs (tessa_replay.rs:1474-1600)."""
import numpy as np
import pytest

from shear_amd import replay as R
from shear_amd.tessa import compact_batches_from_slices, sq_int8_padded_dim


def test_pair_and_payload_formulas_are_exact():
    # tessa_replay.rs:1474-1489
    assert R.tessa_assignment_pairs([(3, 2), (2, 3)]) == 12
    assert R.tessa_leaf_pairs([4, 3]) == 18
    assert R.tessa_fp32_logical_payload_bytes(7, 16) == 476
    assert R.tessa_sq8_logical_payload_bytes(7, 16) == 168


def test_overlap_percentiles_and_exact_fraction_are_exact():
    # tessa_replay.rs:1491-1530
    ref = [1, 2, 3, 4, 5, 6, 7, 8]
    act = [1, 2, 4, 9, 5, 10, 7, 8]
    blocks = [R.TessaCandidateBlock(2 * i, 1, 2, i + 1) for i in range(4)]
    s = R.tessa_overlap_summary(ref, act, blocks)
    assert s.task_count == 4
    assert s.macro_mean == 0.75 and s.pair_weighted_mean == 0.75
    assert (s.p5, s.p50, s.p95) == (0.5, 0.5, 1.0)
    assert s.exact_task_fraction == 0.5


def test_nearest_rank_median_range_and_rotation_are_exact():
    # tessa_replay.rs:1532-1556
    v = [9.0, 1.0, 5.0, 3.0, 7.0]
    assert R.tessa_nearest_rank_percentile(v, 0.05) == 1.0
    assert R.tessa_nearest_rank_percentile(v, 0.50) == 5.0
    assert R.tessa_nearest_rank_percentile(v, 0.95) == 9.0
    assert R.tessa_distribution_summary([4.0, 1.0, 3.0, 2.0]) == R.TessaDistributionSummary(2.5, 1.0, 4.0)
    assert R.tessa_rotated_mode_order(0) == R.ALL_MODES
    assert R.tessa_rotated_mode_order(1) == R.ALL_MODES[1:] + R.ALL_MODES[:1]
    assert R.tessa_rotated_mode_order(6) == R.ALL_MODES


def test_formal_contract_is_strict():
    # tessa_replay.rs:1558-1580
    R.TessaReplayRunConfig(seed=42).validate()
    with pytest.raises(ValueError):
        R.TessaReplayRunConfig(seed=42, warmup_sweeps=4).validate()
    with pytest.raises(ValueError):
        R.TessaReplayRunConfig(seed=42, measured_sweeps=19).validate()
    with pytest.raises(ValueError):
        R.TessaReplayRunConfig(seed=0).validate()


def test_percentile_input_validation():
    with pytest.raises(ValueError):
        R.tessa_nearest_rank_percentile([], 0.5)
    with pytest.raises(ValueError):
        R.tessa_nearest_rank_percentile([1.0], 1.5)
    with pytest.raises(ValueError):
        R.tessa_distribution_summary([float("nan")])


def test_executor_codes_match_reference_modes():
    assert R.TessaReplayMode.A2_SQ8_DP4A_BATCH1.leaf_executor_code == 1
    assert R.TessaReplayMode.A3_SQ8_WMMA_BATCH8.leaf_executor_code == 2
    assert R.TessaReplayMode.SQ8_DP4A_BATCH8.leaf_executor_code is None
    assert R.TessaReplayMode.A3_SQ8_WMMA_BATCH8.assignment_ticket_batch == 8


def test_padded_dim():
    assert sq_int8_padded_dim(768) == 768
    assert sq_int8_padded_dim(100) == 112
    assert sq_int8_padded_dim(3, 8) == 8
    with pytest.raises(ValueError):
        sq_int8_padded_dim(0)


def test_compact_batches_from_slices_uses_min_k_and_stride():
    # compute_backend.rs:32243-32339: row stride max_k, k = min(leaf_knn, size-1)
    gids = np.array([100, 101, 102, 103, 104], np.uint32)
    leaf_rows = np.array([4, 0, 2, 1, 3], np.uint32)
    starts = np.array([0, 2], np.uint64)
    sizes = np.array([2, 3], np.uint64)
    max_k = 4
    ids = np.arange(5 * max_k, dtype=np.uint32)
    d = ids.astype(np.float32) / 10
    b = compact_batches_from_slices(gids, leaf_rows, starts, sizes, ids, d, max_k, leaf_knn=3)
    assert [x.k for x in b] == [1, 2]
    assert b[0].point_ids.tolist() == [104, 100]
    assert b[0].topk_ids.tolist() == [0, 4]
    assert b[1].point_ids.tolist() == [102, 101, 103]
    assert b[1].topk_ids.tolist() == [8, 9, 12, 13, 16, 17]
    with pytest.raises(ValueError):
        compact_batches_from_slices(gids, leaf_rows, np.array([4], np.uint64), np.array([3], np.uint64), ids, d,
                                    max_k, 3)
