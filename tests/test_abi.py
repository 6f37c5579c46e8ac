"""The C-ABI library loads without a GPU, exports every function declared in
include/gs3d_hip.h, and the ctypes structs match the C layout."""

import ctypes
import os
import re
import subprocess

import pytest

from dsl_splat_amd.runtime import abi, native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gs3d_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gs3d_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = native.load()
    declared = _declared_functions()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in gs3d_hip.h but not exported"
        assert name in abi.FUNCTIONS, f"{name} has no ctypes signature"
    assert lib.gs3d_abi_version() == abi.ABI_VERSION
    # Size queries need no device.
    assert native.query("gs3d_sort_scratch_bytes", 1 << 20) > 0
    assert native.query("gs3d_scan_scratch_bytes", 0) >= 0
    assert native.query("gs3d_order_rows_scratch_bytes", 1000) > 0
    assert native.query("gs3d_bin_rows_scratch_bytes", 10_000, 4, 1920, 1080, 0) > 0
    assert native.query("gs3d_bin_rows_scratch_bytes", 10_000, 4, 1920, 1080, 2) > \
        native.query("gs3d_bin_rows_scratch_bytes", 10_000, 4, 1920, 1080, 0)


def test_early_group_item_entry_points_check_their_arguments():
    lib = native.load()
    a = abi.BinArgs()
    a.n, a.views, a.width, a.height = 10, 1, 64, 64
    a.group_pairs = 100
    # AccuTile items carry tile masks: not emitted early.
    a.tile_mode = abi.TILE_MODES["accutile"]
    assert lib.gs3d_emit_group_items(ctypes.byref(a), None, 0, None) == abi.GS3D_ERR_UNSUPPORTED
    assert lib.gs3d_bin_emitted_rows(ctypes.byref(a), None, 0, None) == abi.GS3D_ERR_ARGUMENT
    a.tile_mode = abi.TILE_MODES["radius"]
    # Missing inputs, then a scratch smaller than the capacity needs.
    assert lib.gs3d_emit_group_items(ctypes.byref(a), None, 0, None) == abi.GS3D_ERR_ARGUMENT
    a.centers = a.radii = a.order = a.group_offsets = ctypes.c_void_p(256)
    need = native.query("gs3d_bin_rows_scratch_bytes", 100, 1, 64, 64, 0)
    assert lib.gs3d_emit_group_items(ctypes.byref(a), ctypes.c_void_p(256), need - 1, None) == abi.GS3D_ERR_SCRATCH
    a.group_pairs = 1 << 31
    assert lib.gs3d_emit_group_items(ctypes.byref(a), ctypes.c_void_p(256), need, None) == abi.GS3D_ERR_OVERFLOW
    a.group_pairs = -1
    assert lib.gs3d_emit_group_items(ctypes.byref(a), ctypes.c_void_p(256), need, None) == abi.GS3D_ERR_ARGUMENT


def test_argument_errors_are_reported_without_launching():
    lib = native.load()
    # Invalid sizes are rejected on the host (no device needed).
    assert lib.gs3d_camera_prepare(None, None, -1, 10, 10, 0, None, None, None, None, None) == abi.GS3D_ERR_ARGUMENT
    assert lib.gs3d_sort_pairs_u64(None, None, 10, 70, None, 0, None) == abi.GS3D_ERR_ARGUMENT
    assert lib.gs3d_sort_pairs_u32(None, None, 10, 33, None, 0, None) == abi.GS3D_ERR_ARGUMENT
    assert lib.gs3d_scan_i32(None, -5, None, None, None, 0, None) == abi.GS3D_ERR_ARGUMENT
    args = abi.RenderArgs()
    args.width, args.height, args.views, args.n = 16, 16, 1, 1
    # Any channel count is blended (in windows of up to 64 channels), but an
    # empty channel vector is an argument error.
    args.feat_channels, args.one_tail = 0, 0
    args.ranges = args.centers = args.conics = args.features = ctypes.c_void_p(256)
    assert lib.gs3d_render_fwd(ctypes.byref(args), None) == abi.GS3D_ERR_ARGUMENT
    args.one_tail = 1
    # Statistics: 1..8 requests, kind bits only for existing requests, outputs
    # present for each kind requested.
    args.feat_channels = 3
    st = abi.RenderStatsArgs()
    st.pixel_values = st.counts = st.sums = ctypes.c_void_p(256)
    for requests, mask in ((0, 0), (abi.MAX_STATISTICS + 1, 0), (2, 0b100)):
        st.requests, st.sum_mask = requests, mask
        assert lib.gs3d_render_fwd_stats(ctypes.byref(args), ctypes.byref(st), None) == abi.GS3D_ERR_ARGUMENT
    st.requests, st.sum_mask, st.sums = 2, 0b10, None
    assert lib.gs3d_render_fwd_stats(ctypes.byref(args), ctypes.byref(st), None) == abi.GS3D_ERR_ARGUMENT
    assert lib.gs3d_render_fwd_stats(ctypes.byref(args), None, None) == abi.GS3D_ERR_ARGUMENT
    # Capped lists: a capped blend must be given its overflow flags; a redo
    # blend (which skips tiles) can neither clear a buffer nor total
    # statistics, and neither can a capped one.
    args.final_t = args.contributors = args.image = args.image_alpha = ctypes.c_void_p(256)
    args.caps = ctypes.c_void_p(256)
    assert lib.gs3d_render_fwd(ctypes.byref(args), None) == abi.GS3D_ERR_ARGUMENT
    args.redo = ctypes.c_void_p(256)
    assert lib.gs3d_render_fwd(ctypes.byref(args), None) == abi.GS3D_ERR_ARGUMENT  # no redo_list
    st.requests, st.sum_mask, st.sums = 1, 0b1, ctypes.c_void_p(256)
    args.redo_list = ctypes.c_void_p(256)
    assert lib.gs3d_render_fwd_stats(ctypes.byref(args), ctypes.byref(st), None) == abi.GS3D_ERR_ARGUMENT
    args.caps = args.redo = None
    args.redo_pass = 1
    args.zero_out, args.zero_count = ctypes.c_void_p(256), 4
    assert lib.gs3d_render_fwd(ctypes.byref(args), None) == abi.GS3D_ERR_ARGUMENT
    args.zero_out, args.zero_count = None, 0
    assert lib.gs3d_render_fwd_stats(ctypes.byref(args), ctypes.byref(st), None) == abi.GS3D_ERR_ARGUMENT
    assert lib.gs3d_render_pair_counts(ctypes.byref(args), ctypes.c_void_p(256), None) == abi.GS3D_ERR_ARGUMENT
    args.redo_pass, args.stop_out = 0, ctypes.c_void_p(256)
    assert lib.gs3d_render_fwd_stats(ctypes.byref(args), ctypes.byref(st), None) == abi.GS3D_ERR_ARGUMENT
    assert lib.gs3d_render_pair_counts(ctypes.byref(args), ctypes.c_void_p(256), None) == abi.GS3D_ERR_ARGUMENT
    args.redo_pass, args.stop_out = 1, None
    args.redo_list = None
    assert lib.gs3d_render_fwd(ctypes.byref(args), None) == abi.GS3D_ERR_ARGUMENT
    args.redo_pass = 0
    args.final_t = args.contributors = args.image = args.image_alpha = None
    # Camera keys are 8-byte aligned.
    p = ctypes.c_void_p(256)
    assert lib.gs3d_camera_prepare_keyed(p, p, 1, 10, 10, 0, p, None, None, p, ctypes.c_void_p(260),
                                         None) == abi.GS3D_ERR_ARGUMENT
    # The blend VJP's gradient row strides feed 32-bit multipliers: a stride
    # of 2^31 or more is rejected before any launch.
    bwd = abi.RenderBwdArgs()
    bwd.fwd = args
    bwd.fwd.final_t = bwd.fwd.contributors = ctypes.c_void_p(256)
    bwd.grad_centers = bwd.grad_conics = ctypes.c_void_p(256)
    bwd.grad_centers_stride, bwd.grad_conics_stride = 1 << 31, 4
    assert lib.gs3d_render_bwd(ctypes.byref(bwd), None) == abi.GS3D_ERR_ARGUMENT
    # Zero-size work is a no-op.
    assert lib.gs3d_pair_tiles(None, 0, None, 0, None) == abi.GS3D_OK
    args = abi.BinArgs()
    args.n, args.views, args.width, args.height = 10, 1, 16, 16
    args.group_pairs, args.tile_pairs = 1 << 31, 5
    args.ranges = ctypes.c_void_p(256)
    assert lib.gs3d_bin_rows(ctypes.byref(args), None, 0, None) == abi.GS3D_ERR_OVERFLOW
    p = ctypes.c_void_p(256)
    assert lib.gs3d_bin_redo(ctypes.byref(args), p, p, None, 0, None) == abi.GS3D_ERR_OVERFLOW
    assert lib.gs3d_bin_redo(ctypes.byref(args), None, p, None, 0, None) == abi.GS3D_ERR_ARGUMENT
    assert lib.gs3d_bin_redo(ctypes.byref(args), p, None, None, 0, None) == abi.GS3D_ERR_ARGUMENT
    assert lib.gs3d_bin_redo(None, p, p, None, 0, None) == abi.GS3D_ERR_ARGUMENT
    args.group_pairs = 5
    assert lib.gs3d_bin_redo(ctypes.byref(args), p, p, p, 1, None) == abi.GS3D_ERR_ARGUMENT  # no ids
    args.ids = p
    assert lib.gs3d_bin_redo(ctypes.byref(args), p, p, p, 1, None) == abi.GS3D_ERR_SCRATCH
    with pytest.raises(native.NativeLibraryError, match="invalid argument"):
        native.call("gs3d_scan_i32", None, -1, None, None, None, 0, None)
    # The allocation-free sort rejects counts beyond its static scratch before
    # touching a device (the pointers are never dereferenced).
    big = 300_000_000
    assert native.query("gs3d_sort_scratch_bytes", big) > abi.STATIC_SCRATCH_BYTES
    # The documented limit of the static scratch.
    assert native.query("gs3d_sort_scratch_bytes", 133_693_440) <= abi.STATIC_SCRATCH_BYTES
    assert native.query("gs3d_sort_scratch_bytes", 133_693_441) > abi.STATIC_SCRATCH_BYTES
    assert lib.gs3d_sort_pairs_u64_static(ctypes.c_void_p(256), ctypes.c_void_p(256), big, 45,
                                          None) == abi.GS3D_ERR_SCRATCH
    assert b"GS3D_STATIC_SCRATCH_BYTES" in lib.gs3d_last_error()
    assert lib.gs3d_sort_pairs_u64_static(None, None, 1000, 45, None) == abi.GS3D_ERR_ARGUMENT
    assert lib.gs3d_sort_pairs_u64_static(None, None, 1, 45, None) == abi.GS3D_OK


def test_struct_layout_matches_header(tmp_path):
    prog = ["#include <stdio.h>", "#include <stddef.h>", '#include "gs3d_hip.h"', "int main(void) {"]
    for cname, cls in abi.STRUCTS.items():
        prog.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            prog.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    prog.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(prog))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    c_layout = {}
    for line in out:
        if line:
            struct, field, value = line.split()
            c_layout[(struct, field)] = int(value)
    for cname, cls in abi.STRUCTS.items():
        assert c_layout[(cname, "size")] == ctypes.sizeof(cls), cname
        for field, _ in cls._fields_:
            assert c_layout[(cname, field)] == getattr(cls, field).offset, (cname, field)
