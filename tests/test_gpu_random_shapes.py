"""Layer parity on randomly drawn shapes (fixed seeds).

Each case draws T around every path threshold (few-token, decode, grouped GEMMs,
the multi-workgroup dispatch), d, E, k, I, the shared expert's size (or none) and
group masks, and checks glm_moe_forward against the oracle: the margin-aware
index check, route weights to f32 rounding and the layer output to the rel-L2
bar on the rows whose route matches.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_oracle as O
from livglm_amd.workloads import MoEShape, make_layer

from test_gpu_parity import REL_L2, _check_indices, _oracle_layer, gu  # noqa: F401 (fixture)

_TS = [1, 2, 3, 4, 5, 8, 9, 15, 16, 17, 31, 32, 33, 47, 63, 64, 65, 100, 129, 255, 256, 300, 513]


def _draw(seed: int) -> MoEShape:
    rng = np.random.default_rng(seed)
    T = int(rng.choice(_TS))
    d = int(rng.choice([512, 1024, 1536, 2048, 3072, 4096]))
    E = int(rng.choice([8, 16, 24, 32, 64, 96, 128, 160, 256]))
    k = int(rng.integers(1, min(8, E) + 1))
    I = int(rng.choice([128, 256, 384, 512, 768, 1024]))
    Is = int(rng.choice([0, 128, 256, 512, 768]))
    ng = 1
    for g in (8, 4, 2):
        if E % g == 0 and E // g >= 2 and rng.random() < 0.3:
            ng = g
            break
    tg = int(rng.integers(1, ng + 1)) if ng > 1 else 1
    if tg * (E // ng) < k:
        tg = ng
    while T * d * max(I, Is, 1) > (1 << 27) and T > 1:  # the oracle stays within a second
        T //= 2
    return MoEShape("random", T, d, E, k, I, Is, n_group=ng, topk_group=tg)


def test_draws_cover_the_paths():
    # the fixed seeds reach the few-token, decode and grouped paths, with and
    # without a shared expert and group masks
    shapes = [_draw(s) for s in range(24)]
    Ts = [s.T for s in shapes]
    assert min(Ts) <= 4 and any(16 < t <= 64 for t in Ts) and max(Ts) > 64
    assert any(s.I_shared == 0 for s in shapes) and any(s.I_shared > 0 for s in shapes)
    assert any(s.n_group > 1 for s in shapes)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(24))
def test_moe_layer_random_shape(gu, seed):
    shape = _draw(seed)
    layer = make_layer(shape, 1000 + seed)
    shared = shape.I_shared > 0
    want, inter = _oracle_layer(layer, shape, shared=shared)
    out, w, idx = gu.run_layer(gu.upload_layer(layer), shape, shared=shared)
    got_idx = gu.host(idx).astype(np.uint32)
    _check_indices(got_idx, inter["indices"], inter["choice"], shape.k)
    same = np.all(got_idx == inter["indices"], axis=1)
    assert same.sum() >= shape.T - 1
    np.testing.assert_allclose(gu.host(w)[same], inter["weights"][same], rtol=2e-6, atol=1e-7)
    assert O.rel_l2(gu.host(out)[same], want[same]) < REL_L2
