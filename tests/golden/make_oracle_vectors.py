"""Write the oracle regression vectors of tests/golden/ (run from the repo root):

    python tests/golden/make_oracle_vectors.py

The reference (Python + NVIDIA Warp) cannot run in this environment and ships
no test vectors, so these fixtures are the CPU oracle's own outputs on two
tiny seeded scenes (RGB features; SH degree 3 with absgrad).  They pin the
oracle against accidental change; tests/test_oracle_*.py pin it against
closed forms, brute force and finite differences.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

import oracle  # noqa: E402
from dsl_splat_amd import synthetic  # noqa: E402
from oracle_pipeline import run  # noqa: E402

SCENES = {
    "oracle_rgb_small": dict(name="small", n=300, width=64, height=48, seed=21),
    "oracle_sh3_small": dict(name="sh3_720p", n=300, width=64, height=48, seed=22),
}


def scene_inputs(key):
    cfg = dict(SCENES[key])
    scene = synthetic.make_scene(cfg.pop("name"), **cfg)
    npy = lambda t: None if t is None else t.detach().cpu().numpy().astype(np.float32)
    return dict(
        means=npy(scene.means), quats=npy(torch.nn.functional.normalize(scene.quats, dim=-1)),
        scales=npy(scene.scales), opacities=npy(scene.opacities), viewmats=npy(scene.viewmats),
        Ks=npy(scene.Ks), width=scene.width, height=scene.height, features=npy(scene.features),
        sh=npy(scene.sh_coeffs), sh_degree=scene.sh_degree, upstream=npy(scene.loss_weights),
        absgrad=bool(scene.absgrad),
    )


def outputs(inp):
    out = run(inp["means"], inp["quats"], inp["scales"], inp["opacities"], inp["viewmats"], inp["Ks"],
              inp["width"], inp["height"], features=inp["features"], sh=inp["sh"], sh_degree=inp["sh_degree"],
              upstream=inp["upstream"], absgrad=inp["absgrad"])
    p, g, pg = out["proj"], out["render_grads"], out["proj_grads"]
    res = dict(radii=p["radii"], tiles=p["tiles"], centers=p["centers"], conics=p["conics"], depths=p["depths"],
               sorted_keys=out["sorted_keys"], sorted_vals=out["sorted_vals"], ranges=out["ranges"],
               image=out["image"], final_t=out["final_t"], contributors=out["contributors"],
               grad_centers=g["centers"], grad_conics=g["conics"], grad_features=g["features"],
               grad_means=pg["means"], grad_quats=pg["quats"], grad_scales=pg["scales"],
               grad_opacities=pg["opacities"], grad_viewmats=out["grad_viewmats"])
    if inp["sh"] is not None:
        res["colors"] = p["colors"]
        res["grad_sh"] = pg["sh"]
    return res


def main():
    oracle.build()
    oracle.set_threads(1)
    for key in SCENES:
        inp = scene_inputs(key)
        res = outputs(inp)
        arrays = {f"in_{k}": np.asarray(v) for k, v in inp.items() if v is not None}
        arrays.update({f"out_{k}": np.asarray(v) for k, v in res.items()})
        path = os.path.join(HERE, key + ".npz")
        np.savez_compressed(path, **arrays)
        print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
