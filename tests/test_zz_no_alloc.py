"""gs3d_sort_pairs_u64_static, the allocation-free pair sort, against
gs3d_sort_pairs_u64 (caller scratch) through the C-ABI: bit-identical keys
and values on two calls in a row, the second smaller (the static scratch
keeps the first call's contents)."""

import ctypes

import numpy as np
import pytest
import torch

from dsl_splat_amd.runtime import abi, native

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _pairs(count, seed):
    g = torch.Generator().manual_seed(seed)
    tiles = torch.randint(0, 8160, (count,), generator=g, dtype=torch.int64)
    depth = torch.rand(count, generator=g) * 6 + 1
    keys = (tiles << 32) | depth.view(torch.int32).to(torch.int64)
    keys[1::2] = keys[0::2][: len(keys[1::2])]  # ties: stability matters
    values = torch.arange(count, dtype=torch.int32)
    return keys, values


def _sort(keys, values, end_bit, static):
    count = keys.numel()
    k = torch.empty(2 * count, dtype=torch.int64, device=DEV)
    v = torch.empty(2 * count, dtype=torch.int32, device=DEV)
    k[:count] = keys.to(DEV)
    v[:count] = values.to(DEV)
    stream = native.stream(k.device)
    if static:
        native.call("gs3d_sort_pairs_u64_static", native.ptr(k), native.ptr(v), count, end_bit, stream)
    else:
        scratch = torch.empty(native.query("gs3d_sort_scratch_bytes", count), dtype=torch.uint8, device=DEV)
        native.call("gs3d_sort_pairs_u64", native.ptr(k), native.ptr(v), count, end_bit, native.ptr(scratch),
                    scratch.numel(), stream)
    torch.cuda.synchronize()
    return k[:count].cpu(), v[:count].cpu()


def test_static_sort_matches_scratch_sort():
    for count, seed in ((1_500_003, 1), (200_001, 2)):
        print(f"static sort count={count}", flush=True)
        keys, values = _pairs(count, seed)
        end_bit = 32 + 14
        ks, vs = _sort(keys, values, end_bit, static=True)
        kr, vr = _sort(keys, values, end_bit, static=False)
        assert torch.equal(ks, kr) and torch.equal(vs, vr)
        # Stable order by the low end_bit key bits.
        masked = keys.numpy() & ((1 << end_bit) - 1)
        order = np.argsort(masked, kind="stable")
        np.testing.assert_array_equal(vs.numpy(), values.numpy()[order])
