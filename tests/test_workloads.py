"""CPU checks of the synthetic workload generators (routing biases)."""

from __future__ import annotations

import numpy as np

from livglm_amd.workloads import SHAPES, markov_bias_trace, zipf_bias


def test_markov_trace_forces_k_experts_and_keeps_seventy_percent():
    E, k, layers, steps = 128, 8, 6, 200
    tr = markov_bias_trace(E, k, layers, steps, np.random.default_rng(3))
    assert tr.shape == (steps, layers, E) and tr.dtype == np.float32
    chosen = tr > 0
    assert np.all(chosen.sum(axis=2) == k)
    # boost dominates any sigmoid score (< 1) plus a zero bias
    assert np.all(tr[chosen] >= 10.0) and np.all(tr[~chosen] == 0.0)
    kept = (chosen[1:] & chosen[:-1]).sum(axis=2)  # experts shared with the previous step
    frac = kept.sum() / (k * layers * (steps - 1))
    assert abs(frac - 0.7) < 0.03


def test_zipf_bias_profile():
    rng = np.random.default_rng(5)
    b = zipf_bias(128, rng)
    ranked = np.sort(b)[::-1]
    np.testing.assert_allclose(ranked, np.arange(1, 129, dtype=np.float64) ** -1.1, rtol=1e-6)


def test_stack_shape_geometry():
    s = SHAPES["stack42_t1"]
    assert (s.layers, s.steps, s.T, s.k) == (42, 256, 1, 8)
    assert s.expert_bytes == 2_506_752
    assert s.layers * s.k * s.expert_bytes == 842_268_672
