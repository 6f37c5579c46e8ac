"""ctypes mirror of the argument structs declared in include/gs3d_hip.h.

The field order and types must match the C header exactly; a CPU test
compiles the header and compares every offset with the ones below.
"""

import ctypes

c_float_p = ctypes.POINTER(ctypes.c_float)
c_int32_p = ctypes.POINTER(ctypes.c_int32)

ABI_VERSION = 10

# Tile modes (GS3D_TILE_*), named as the reference's TileMode literals.
TILE_MODES = {"radius": 0, "snugbox": 1, "accutile": 2}

GS3D_OK = 0
GS3D_ERR_ARGUMENT = -1
GS3D_ERR_LAUNCH = -2
GS3D_ERR_UNSUPPORTED = -3
GS3D_ERR_SCRATCH = -4
GS3D_ERR_OVERFLOW = -5
# Static scratch of gs3d_sort_pairs_u64_static (GS3D_STATIC_SCRATCH_BYTES).
STATIC_SCRATCH_BYTES = 128 << 20

STATUS_NAMES = {
    GS3D_ERR_ARGUMENT: "invalid argument",
    GS3D_ERR_LAUNCH: "kernel launch failed",
    GS3D_ERR_UNSUPPORTED: "unsupported configuration",
    GS3D_ERR_SCRATCH: "scratch buffer too small",
    GS3D_ERR_OVERFLOW: "pair count exceeds int32 offsets",
}

_P = ctypes.c_void_p


class ProjectArgs(ctypes.Structure):
    _fields_ = [
        ("n", ctypes.c_int32),
        ("views", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("height", ctypes.c_int32),
        ("near_plane", ctypes.c_float),
        ("far_plane", ctypes.c_float),
        ("radius_clip", ctypes.c_float),
        ("means", _P),
        ("quats", _P),
        ("scales", _P),
        ("opacities", _P),
        ("view", _P),
        ("projection", _P),
        ("intrinsics", _P),
        ("centers", _P),
        ("conics", _P),
        ("radii", _P),
        ("tiles", _P),
        ("depths", _P),
        ("sh", _P),
        ("sh_view_stride", ctypes.c_int64),
        ("sh_rows", ctypes.c_int32),
        ("sh_degree", ctypes.c_int32),
        ("camera_centers", _P),
        ("colors", _P),
        ("means2d", _P),
        ("meta_opacities", _P),
        ("meta_conics", _P),
        ("tile_mode", ctypes.c_int32),
        ("normalize_quats", ctypes.c_int32),
    ]


class ProjectBwdArgs(ctypes.Structure):
    _fields_ = [
        ("n", ctypes.c_int32),
        ("views", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("height", ctypes.c_int32),
        ("means", _P),
        ("quats", _P),
        ("scales", _P),
        ("opacities", _P),
        ("view", _P),
        ("projection", _P),
        ("intrinsics", _P),
        ("radii", _P),
        ("grad_centers", _P),
        ("grad_centers_stride", ctypes.c_int64),
        ("grad_conics", _P),
        ("grad_conics_stride", ctypes.c_int64),
        ("grad_means", _P),
        ("grad_quats", _P),
        ("grad_scales", _P),
        ("grad_opacities", _P),
        ("grad_view", _P),
        ("grad_projection", _P),
        ("sh", _P),
        ("sh_view_stride", ctypes.c_int64),
        ("sh_rows", ctypes.c_int32),
        ("sh_degree", ctypes.c_int32),
        ("camera_centers", _P),
        ("grad_colors", _P),
        ("grad_colors_stride", ctypes.c_int64),
        ("grad_sh", _P),
        ("grad_camera_centers", _P),
        ("normalize_quats", ctypes.c_int32),
        ("screen_grad", ctypes.c_void_p),
    ]


class EmitArgs(ctypes.Structure):
    _fields_ = [
        ("n", ctypes.c_int32),
        ("views", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("height", ctypes.c_int32),
        ("centers", _P),
        ("radii", _P),
        ("depths", _P),
        ("offsets", _P),
        ("keys", _P),
        ("values", _P),
        ("conics", _P),
        ("tile_mode", ctypes.c_int32),
    ]


class OrderArgs(ctypes.Structure):
    _fields_ = [
        ("n", ctypes.c_int32),
        ("views", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("height", ctypes.c_int32),
        ("depths", _P),
        ("centers", _P),
        ("radii", _P),
        ("order", _P),
        ("group_offsets", _P),
        ("totals", _P),
        ("conics", _P),
        ("tile_mode", ctypes.c_int32),
        ("tiles_out", _P),
        ("footprints", _P),
        ("sort_bits", ctypes.c_int32),
        ("key_bits_out", _P),
    ]


class BinArgs(ctypes.Structure):
    _fields_ = [
        ("n", ctypes.c_int32),
        ("views", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("height", ctypes.c_int32),
        ("centers", _P),
        ("radii", _P),
        ("order", _P),
        ("group_offsets", _P),
        ("group_pairs", ctypes.c_int64),
        ("tile_pairs", ctypes.c_int64),
        ("ranges", _P),
        ("ids", _P),
        ("conics", _P),
        ("tile_mode", ctypes.c_int32),
        ("footprints", _P),
        ("caps", _P),
        ("redo_list", _P),
    ]


class RenderArgs(ctypes.Structure):
    _fields_ = [
        ("width", ctypes.c_int32),
        ("height", ctypes.c_int32),
        ("views", ctypes.c_int32),
        ("n", ctypes.c_int32),
        ("ranges", _P),
        ("ids", _P),
        ("centers", _P),
        ("conics", _P),
        ("features", _P),
        ("feat_channels", ctypes.c_int32),
        ("feat_stride", ctypes.c_int64),
        ("feat_view_stride", ctypes.c_int64),
        ("extra", _P),
        ("extra_channels", ctypes.c_int32),
        ("extra_stride", ctypes.c_int64),
        ("extra_view_stride", ctypes.c_int64),
        ("one_tail", ctypes.c_int32),
        ("background", _P),
        ("background_view_stride", ctypes.c_int64),
        ("image", _P),
        ("image_extra", _P),
        ("image_alpha", _P),
        ("final_t", _P),
        ("contributors", _P),
        ("zero_out", _P),
        ("zero_count", ctypes.c_int64),
        ("caps", _P),
        ("stop_out", _P),
        ("redo", _P),
        ("redo_list", _P),
        ("redo_pass", ctypes.c_int32),
    ]


MAX_STATISTICS = 8


class RenderStatsArgs(ctypes.Structure):
    _fields_ = [
        ("requests", ctypes.c_int32),
        ("sum_mask", ctypes.c_uint32),
        ("pixel_values", _P),
        ("pixel_view_stride", ctypes.c_int64),
        ("counts", _P),
        ("counts_view_stride", ctypes.c_int64),
        ("sums", _P),
        ("sums_view_stride", ctypes.c_int64),
    ]


class RenderBwdArgs(ctypes.Structure):
    _fields_ = [
        ("fwd", RenderArgs),
        ("upstream", _P),
        ("upstream_stride", ctypes.c_int64),
        ("upstream_extra", _P),
        ("upstream_extra_stride", ctypes.c_int64),
        ("upstream_alpha", _P),
        ("upstream_alpha_stride", ctypes.c_int64),
        ("grad_centers", _P),
        ("grad_centers_stride", ctypes.c_int64),
        ("grad_conics", _P),
        ("grad_conics_stride", ctypes.c_int64),
        ("abs_centers", _P),
        ("abs_stride", ctypes.c_int64),
        ("grad_features", _P),
        ("grad_feat_stride", ctypes.c_int64),
        ("grad_feat_view_stride", ctypes.c_int64),
        ("grad_extra", _P),
        ("grad_extra_stride", ctypes.c_int64),
        ("grad_extra_view_stride", ctypes.c_int64),
    ]


STRUCTS = {
    "gs3d_project_args": ProjectArgs,
    "gs3d_project_bwd_args": ProjectBwdArgs,
    "gs3d_emit_args": EmitArgs,
    "gs3d_order_args": OrderArgs,
    "gs3d_bin_args": BinArgs,
    "gs3d_render_args": RenderArgs,
    "gs3d_render_stats_args": RenderStatsArgs,
    "gs3d_render_bwd_args": RenderBwdArgs,
}

# Exported functions: name -> (restype, argtypes).  void* carries device
# pointers and the hipStream_t.
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t

FUNCTIONS = {
    "gs3d_abi_version": (ctypes.c_int, []),
    "gs3d_last_error": (ctypes.c_char_p, []),
    "gs3d_camera_prepare": (
        ctypes.c_int,
        [_P, _P, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P],
    ),
    "gs3d_camera_prepare_keyed": (
        ctypes.c_int,
        [_P, _P, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P],
    ),
    "gs3d_camera_backward": (
        ctypes.c_int,
        [_P, _P, _I32, _I32, _P, _P, _I32, _P, _P],
    ),
    "gs3d_project_fwd": (ctypes.c_int, [ctypes.POINTER(ProjectArgs), _P]),
    "gs3d_project_bwd": (ctypes.c_int, [ctypes.POINTER(ProjectBwdArgs), _P]),
    "gs3d_sh_fwd": (ctypes.c_int, [_P, _I32, _P, _P, _I32, _I32, _P, _P, _P]),
    "gs3d_sh_bwd": (
        ctypes.c_int,
        [_P, _I32, _P, _P, _P, _P, _I32, _I32, _P, _P, _P],
    ),
    "gs3d_metadata": (ctypes.c_int, [_P, _P, _P, _I64, _P, _P, _P, _P]),
    "gs3d_scan_scratch_bytes": (_SZ, [_I64]),
    "gs3d_scan_i32": (ctypes.c_int, [_P, _I64, _P, _P, _P, _SZ, _P]),
    "gs3d_emit_scratch_bytes": (_SZ, [_I64]),
    "gs3d_emit_keys": (ctypes.c_int, [ctypes.POINTER(EmitArgs), _P, _SZ, _P]),
    "gs3d_sort_scratch_bytes": (_SZ, [_I64]),
    "gs3d_sort_pairs_u64": (ctypes.c_int, [_P, _P, _I64, _I32, _P, _SZ, _P]),
    "gs3d_sort_pairs_u64_static": (ctypes.c_int, [_P, _P, _I64, _I32, _P]),
    "gs3d_tile_ranges": (ctypes.c_int, [_P, _I64, _P, _I64, _P]),
    "gs3d_order_rows_scratch_bytes": (_SZ, [_I64]),
    "gs3d_order_rows": (ctypes.c_int, [ctypes.POINTER(OrderArgs), _P, _SZ, _P]),
    "gs3d_bin_rows_scratch_bytes": (_SZ, [_I64, _I32, _I32, _I32, _I32]),
    "gs3d_bin_rows": (ctypes.c_int, [ctypes.POINTER(BinArgs), _P, _SZ, _P]),
    "gs3d_emit_group_items": (ctypes.c_int, [ctypes.POINTER(BinArgs), _P, _SZ, _P]),
    "gs3d_bin_emitted_rows": (ctypes.c_int, [ctypes.POINTER(BinArgs), _P, _SZ, _P]),
    "gs3d_bin_redo": (ctypes.c_int, [ctypes.POINTER(BinArgs), _P, _P, _P, _SZ, _P]),
    "gs3d_bin_capped_items": (ctypes.c_int, [ctypes.POINTER(BinArgs), _P, _SZ, _P, _P]),
    "gs3d_pair_tiles": (ctypes.c_int, [_P, _I64, _P, _I64, _P]),
    "gs3d_sort_pairs_u32": (ctypes.c_int, [_P, _P, _I64, _I32, _P, _SZ, _P]),
    "gs3d_expand_keys": (ctypes.c_int, [_P, _P, _I64, _P, _I32, _I32, _P, _P]),
    "gs3d_render_fwd": (ctypes.c_int, [ctypes.POINTER(RenderArgs), _P]),
    "gs3d_render_pair_counts": (ctypes.c_int, [ctypes.POINTER(RenderArgs), _P, _P]),
    "gs3d_render_fwd_stats": (ctypes.c_int, [ctypes.POINTER(RenderArgs), ctypes.POINTER(RenderStatsArgs), _P]),
    "gs3d_render_bwd": (ctypes.c_int, [ctypes.POINTER(RenderBwdArgs), _P]),
}
