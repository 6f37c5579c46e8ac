"""The oracle reproduces its committed regression vectors (tests/golden/,
written by tests/golden/make_oracle_vectors.py): integer outputs exactly,
float outputs to a few ulp (the fixtures may have been written on another
host's libm)."""

import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))

from make_oracle_vectors import SCENES, outputs  # noqa: E402

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _inputs(z):
    get = lambda k: z[f"in_{k}"] if f"in_{k}" in z.files else None
    return dict(means=get("means"), quats=get("quats"), scales=get("scales"), opacities=get("opacities"),
                viewmats=get("viewmats"), Ks=get("Ks"), width=int(get("width")), height=int(get("height")),
                features=get("features"), sh=get("sh"),
                sh_degree=None if get("sh_degree") is None else int(get("sh_degree")),
                upstream=get("upstream"), absgrad=bool(get("absgrad")))


@pytest.mark.parametrize("key", sorted(SCENES))
def test_oracle_matches_golden_vectors(oracle_lib, key):
    with np.load(os.path.join(GOLDEN, key + ".npz")) as z:
        inp = _inputs(z)
        expected = {k[4:]: z[k] for k in z.files if k.startswith("out_")}
    got = outputs(inp)
    assert set(got) == set(expected)
    assert expected["sorted_vals"].size > 0
    for name, ref in expected.items():
        val = np.asarray(got[name])
        assert val.shape == ref.shape, name
        if np.issubdtype(ref.dtype, np.integer):
            np.testing.assert_array_equal(val, ref, err_msg=name)
        else:
            scale = max(1.0, float(np.abs(ref).max()))
            np.testing.assert_allclose(val, ref, rtol=1e-5, atol=1e-6 * scale, err_msg=name)
