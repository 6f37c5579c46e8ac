"""The round-trip smoke check (one small SH3 rasterize forward + backward
with absolute gradients against the oracle) as part of the GPU suite, so the
entry point the smoke run uses stays consistent with the oracle."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.gpu
def test_smoke_entry_point():
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    import __graft_entry__

    __graft_entry__.smoke()
