"""Pins for the oracle's contribution statistics (statistics.py:46-70,
observed at gs3d/render.py:109-115) and the host-side request validation
(statistics.py:73-156).

With one-hot features (Gaussian g blends channel g with value 1) and no
background, channel g of the blended image at pixel p is exactly the blend
weight alpha*T of g at p, and zero where g is not accepted.  Every statistic
is then a closed form of the image, which the float64 renderer pins
(tests/test_oracle_render.py): counts = number of accepted (masked) pixels,
sums = sum of value * weight over them, and the all-ones weighted sum over all
Gaussians equals the alpha channel summed over the image."""

import numpy as np
import pytest
import torch

from dsl_splat_amd import synthetic
from dsl_splat_amd.statistics import MaskedContributionCount, WeightedContributionSum, prepare_statistics
from test_oracle_render import _pipeline


@pytest.mark.parametrize("name,n,W,H,seed", [("small", 40, 48, 40, 3), ("sh3_1080p_4view", 30, 56, 36, 4)])
def test_statistics_are_closed_forms_of_one_hot_blend(oracle_lib, name, n, W, H, seed):
    scene = synthetic.make_scene(name, n=n, width=W, height=H, seed=seed)
    feats = np.eye(n, dtype=np.float32)
    out, ranges, ids, image, final_t, contrib = _pipeline(oracle_lib, scene, features=feats)
    views = image.shape[0]
    rng = np.random.default_rng(seed)
    mask = rng.random((views, H, W)) < 0.5
    weights = rng.standard_normal((views, H, W)).astype(np.float32)
    weights[rng.random((views, H, W)) < 0.2] = 0.0
    ones = np.ones((views, H, W), np.float32)
    # count(mask), sum(weights), sum(ones), count(everywhere): rows are numbered
    # per kind, so counts = [mask, everywhere] and sums = [weights, ones].
    kinds = [0, 1, 1, 0]
    pv = np.stack([mask.astype(np.float32), weights, ones, ones], axis=1)
    img2, ft2, ct2, counts, sums = oracle_lib.render_fwd_stats(W, H, ranges, ids, out["centers"], out["conics"],
                                                               feats, kinds, pv)
    np.testing.assert_array_equal(img2, image)  # statistics change no blend output
    np.testing.assert_array_equal(ft2, final_t)
    np.testing.assert_array_equal(ct2, contrib)
    assert counts.shape == (views, 2, n) and sums.shape == (views, 2, n)
    w = image[..., :n].astype(np.float64)  # (views, H, W, n) blend weights
    accepted = w > 0
    assert accepted.sum() > 100
    np.testing.assert_array_equal(counts[:, 1], accepted.sum((1, 2)))
    np.testing.assert_array_equal(counts[:, 0], (accepted & mask[..., None]).sum((1, 2)))
    np.testing.assert_allclose(sums[:, 1], w.sum((1, 2)), rtol=1e-5, atol=1e-6)
    weighted = w * weights[..., None].astype(np.float64)
    tol = 1e-5 * np.abs(weighted).sum((1, 2)) + 1e-7
    assert np.all(np.abs(sums[:, 0] - weighted.sum((1, 2))) <= tol)
    np.testing.assert_allclose(sums[:, 1].astype(np.float64).sum(-1), image[..., -1].astype(np.float64).sum((1, 2)),
                               rtol=1e-5)


def test_prepare_statistics_layout_and_rows():
    H, W, C, N = 4, 5, 2, 7
    dev = torch.device("cpu")
    m = torch.zeros((H, W), dtype=torch.bool)
    m[1, 2] = True
    wts = torch.arange(C * H * W, dtype=torch.float32).reshape(C, H, W)
    reqs = [WeightedContributionSum("w", wts), MaskedContributionCount("m", m), WeightedContributionSum("w2", wts[0])]
    prepared, results = prepare_statistics(reqs, batch_dims=(), batch_count=1, cameras=C, n=N, width=W, height=H,
                                           device=dev)
    assert len(prepared) == 1
    p = prepared[0]
    assert p.key == (1, 0, 1)
    assert p.pixel_values.shape == (C, 3, H * W) and p.pixel_values.is_contiguous()
    assert torch.equal(p.pixel_values[:, 0], wts.reshape(C, -1))
    assert torch.equal(p.pixel_values[1, 1], m.reshape(-1).float())
    assert torch.equal(p.pixel_values[1, 2], wts[0].reshape(-1))
    assert p.counts.shape == (C, 1, N) and p.sums.shape == (C, 2, N)
    assert set(results) == {"w", "m", "w2"}
    assert all(v.shape == (C, N) for v in results.values())
    # Each result aliases its row of the accumulators.
    p.sums[:, 1] += 3.0
    p.counts[:, 0] += 2
    assert torch.all(results["w2"] == 3.0) and torch.all(results["w"] == 0.0) and torch.all(results["m"] == 2)


def test_prepare_statistics_rejects_bad_requests():
    dev = torch.device("cpu")
    kw = dict(batch_dims=(), batch_count=1, cameras=1, n=3, width=4, height=2, device=dev)
    m = torch.ones((2, 4), dtype=torch.bool)
    with pytest.raises(TypeError):
        prepare_statistics([object()], **kw)
    with pytest.raises(ValueError, match="unique"):
        prepare_statistics([MaskedContributionCount("a", m), MaskedContributionCount("a", m)], **kw)
    with pytest.raises(ValueError, match="unique"):
        prepare_statistics([MaskedContributionCount("", m)], **kw)
    with pytest.raises(ValueError, match="must use"):
        prepare_statistics([MaskedContributionCount("a", m.float())], **kw)
    with pytest.raises(ValueError, match="must use"):
        prepare_statistics([WeightedContributionSum("a", m)], **kw)
    with pytest.raises(ValueError, match="non-differentiable"):
        prepare_statistics([WeightedContributionSum("a", torch.ones((2, 4), requires_grad=True))], **kw)
    with pytest.raises(ValueError, match="shape"):
        prepare_statistics([MaskedContributionCount("a", torch.ones((4, 2), dtype=torch.bool))], **kw)
    with pytest.raises(NotImplementedError):
        prepare_statistics([MaskedContributionCount(f"r{i}", m) for i in range(9)], **kw)
