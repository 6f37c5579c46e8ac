/*
 * gs3d_hip.h — C ABI of the MI355X (gfx950) original-3DGS rasterizer.
 *
 * Every entry point is stateless and reentrant: it takes raw device pointers,
 * element counts, scalar parameters, a hipStream_t (passed as void*) and, where
 * it needs temporary device memory, a caller-provided scratch buffer whose size
 * is returned by the matching *_scratch_bytes query.  No entry point allocates
 * device memory, retains a pointer after it returns, or synchronises the
 * stream.  All launches go to the given stream in submission order.
 *
 * Return value: GS3D_OK (0) or a negative status.  Invalid arguments are
 * detected on the host before anything is launched.
 *
 * Each declaration names the reference launch it replaces (paths relative to
 * the dsl_splat package of YukiNagato/dsl_splat).  Multi-view launches
 * ("views" > 1) are equivalent to one reference launch per view; views are
 * stored back to back with the strides given in the argument structs.
 *
 * Layouts: float32 row-major; matrices (4,4)/(3,3) row-major per view; all
 * per-view Gaussian arrays are (views, N, ...) contiguous unless a stride
 * argument says otherwise.
 */
#ifndef GS3D_HIP_H
#define GS3D_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    GS3D_OK = 0,
    GS3D_ERR_ARGUMENT = -1,   /* bad pointer/size/stride combination */
    GS3D_ERR_LAUNCH = -2,     /* hipGetLastError after a launch */
    GS3D_ERR_UNSUPPORTED = -3,/* channel count or degree outside what was built */
    GS3D_ERR_SCRATCH = -4,    /* scratch buffer smaller than *_scratch_bytes */
    GS3D_ERR_OVERFLOW = -5    /* a count that would not fit int32 offsets */
};

/* ABI revision; bumped whenever a struct layout or signature changes. */
int gs3d_abi_version(void);

/* Last HIP error string seen by this thread (for diagnostics). */
const char* gs3d_last_error(void);

/* ------------------------------------------------------------------------
 * Camera preparation.
 * Replaces splatting/camera_kernels.py:11-66 (prepare_kernel), launched from
 * splatting/cameras.py:45-63.  Per camera i: error code (0 ok, 2 non-finite K
 * or fx,fy<=0, 1 skew/non-pinhole K, 3 singular view with with_centers);
 * full projection rows (count,4,4); with_centers: view inverse (count,4,4) and
 * camera centre inverse[0:3,3] (count,3).
 * ---------------------------------------------------------------------- */
int gs3d_camera_prepare(const float* views, const float* Ks, int32_t count,
                        int32_t width, int32_t height, int32_t with_centers,
                        float* full, float* inverse, float* centers,
                        int32_t* errors, void* stream);

/* gs3d_camera_prepare that also writes keys (count uint64, 8-byte aligned;
 * NULL: none): a 64-bit key of each camera's view matrix and intrinsics,
 * with each value rounded to 12 mantissa bits, so that equal cameras (and
 * poses an optimiser step apart) share a key.  No counterpart in the
 * reference: the rasterizer uses the keys to find the tile-list caps that
 * an earlier frame of the same camera measured (gs3d_render_args.caps). */
int gs3d_camera_prepare_keyed(const float* views, const float* Ks, int32_t count,
                              int32_t width, int32_t height, int32_t with_centers,
                              float* full, float* inverse, float* centers,
                              int32_t* errors, uint64_t* keys, void* stream);

/* Replaces splatting/camera_kernels.py:69-106 (backward_kernel), launched from
 * splatting/cameras.py:98-114.  grad_full and/or grad_centers may be NULL.
 * Writes grad_views (count,4,4) (overwritten, not accumulated). */
int gs3d_camera_backward(const float* Ks, const float* grad_full,
                         int32_t width, int32_t height, const float* inverse,
                         const float* grad_centers, int32_t count,
                         float* grad_views, void* stream);

/* ------------------------------------------------------------------------
 * Projection forward (+ optional fused SH colour and training metadata).
 * Replaces gs3d/projection.py:89-164 (project, launched at :331-353); with
 * sh != NULL also primitives/sh.py:44-79 (evaluate, launched from
 * primitives/spherical_harmonics.py:218-233 with radii masking); with
 * means2d != NULL also splatting/metadata.py:12-31 (_prepare, :296-311).
 * Culled rows get radii = tiles = 0 and zeros in centers/conics/depths.
 * ---------------------------------------------------------------------- */
/* Tile modes (splatting/intersections.py:21-26, gs3d/cameras.py:20-22):
 * RADIUS lists the square of 3-sigma tiles (the original 3DGS rule); SNUGBOX
 * the rectangle of the opacity-aware alpha >= 1/255 ellipse inside it
 * (footprint, intersections.py:46-116); ACCUTILE, per strip of tiles along
 * the shorter side of that rectangle, only the tiles the ellipse crosses
 * (visit, :160-218).  Every mode keeps all pixels the blend accepts. */
#define GS3D_TILE_RADIUS 0
#define GS3D_TILE_SNUGBOX 1
#define GS3D_TILE_ACCUTILE 2

typedef struct gs3d_project_args {
    int32_t n;            /* Gaussians */
    int32_t views;        /* cameras handled by this launch */
    int32_t width, height;
    float near_plane, far_plane, radius_clip;
    const float* means;       /* (N,3) */
    const float* quats;       /* (N,4) wxyz, already normalised */
    const float* scales;      /* (N,3) activated */
    const float* opacities;   /* (N,) activated */
    const float* view;        /* (views,4,4) world->camera */
    const float* projection;  /* (views,4,4) from gs3d_camera_prepare */
    const float* intrinsics;  /* (views,3,3) */
    float* centers;           /* (views,N,2) pixel centres */
    float* conics;            /* (views,N,4) inverse cov (a,b,c) + opacity */
    int32_t* radii;           /* (views,N) */
    int32_t* tiles;           /* (views,N) touched 16x16 tiles */
    float* depths;            /* (views,N) camera-space z */
    /* fused SH (sh == NULL disables) */
    const float* sh;          /* (N,K,3), or per view with sh_view_stride */
    int64_t sh_view_stride;   /* floats between views; 0 = shared by all views */
    int32_t sh_rows;          /* K (row count of each Gaussian's block) */
    int32_t sh_degree;        /* 0..3; (deg+1)^2 <= K */
    const float* camera_centers; /* (views,3); required when sh_degree > 0 */
    float* colors;            /* (views,N,3) */
    /* fused metadata (means2d == NULL disables) */
    float* means2d;           /* (views,N,2) */
    float* meta_opacities;    /* (views,N) */
    float* meta_conics;       /* (views,N,3) */
    int32_t tile_mode;        /* GS3D_TILE_*: what tiles (views,N) counts (projection.py:150-161) */
    int32_t normalize_quats;  /* 1: quats are raw and normalised in the kernel as F.normalize does (inputs.py:252) */
} gs3d_project_args;

int gs3d_project_fwd(const gs3d_project_args* args, void* stream);

/* ------------------------------------------------------------------------
 * Projection backward (+ optional fused SH backward).
 * Replaces gs3d/projection.py:213-285 (project_backward, launched at
 * :393-422) and, with sh != NULL, primitives/sh.py:82-138 (backward, launched
 * from primitives/spherical_harmonics.py:256-273) followed by the Torch
 * "means - camera centre" VJP of gs3d/api.py:160-164.
 * Per-Gaussian outputs are dense, summed over views and overwritten (culled
 * rows give zeros).  grad_view/grad_projection/grad_camera_centers are
 * accumulated with atomics: the caller zeroes them.  Any output may be NULL.
 * ---------------------------------------------------------------------- */
typedef struct gs3d_project_bwd_args {
    int32_t n, views, width, height;
    const float* means;
    const float* quats;
    const float* scales;
    const float* opacities;
    const float* view;        /* (views,4,4) */
    const float* projection;  /* (views,4,4) */
    const float* intrinsics;  /* (views,3,3) */
    const int32_t* radii;     /* (views,N) */
    const float* grad_centers;   /* (views,N,*) rows of grad_centers_stride floats */
    int64_t grad_centers_stride;
    const float* grad_conics;    /* (views,N,*) rows of grad_conics_stride floats (a,b,c,opacity) */
    int64_t grad_conics_stride;
    float* grad_means;        /* (N,3) */
    float* grad_quats;        /* (N,4) */
    float* grad_scales;       /* (N,3) */
    float* grad_opacities;    /* (N,) */
    float* grad_view;         /* (views,4,4) accumulated */
    float* grad_projection;   /* (views,4,4) accumulated */
    /* fused SH backward (sh == NULL disables) */
    const float* sh;
    int64_t sh_view_stride;   /* 0 = shared coefficients; grads then summed over views */
    int32_t sh_rows, sh_degree;
    const float* camera_centers;  /* (views,3) */
    const float* grad_colors;     /* (views,N,*) rows of grad_colors_stride floats */
    int64_t grad_colors_stride;
    float* grad_sh;               /* like sh (dense, rows beyond (deg+1)^2 are zero) */
    float* grad_camera_centers;   /* (views,3) accumulated */
    int32_t normalize_quats;      /* 1: quats are raw; grad_quats is taken through the normalisation */
    /* (views,N,2) contiguous copy of the centre gradients, zero where radii
     * are not positive: the means2d gradient without a strided copy.  May be
     * NULL. */
    float* screen_grad;
} gs3d_project_bwd_args;

int gs3d_project_bwd(const gs3d_project_bwd_args* args, void* stream);

/* ------------------------------------------------------------------------
 * Standalone SH0-3 (primitives/sh.py:44-138 through
 * primitives/spherical_harmonics.py:198-281).  radii may be NULL (no mask).
 * coefficients (N,K,3) with row stride K*3, directions (N,3).
 * active (N,3) uint8 clamp mask may be NULL.
 * ---------------------------------------------------------------------- */
int gs3d_sh_fwd(const float* coefficients, int32_t rows, const float* directions,
                const int32_t* radii, int32_t n, int32_t degree,
                float* colors, uint8_t* active, void* stream);
/* grad_coefficients (N,K,3) fully written (zeros beyond (deg+1)^2), may be
 * NULL; grad_directions (N,3) may be NULL. */
int gs3d_sh_bwd(const float* coefficients, int32_t rows, const float* directions,
                const int32_t* radii, const uint8_t* active, const float* upstream,
                int32_t n, int32_t degree, float* grad_coefficients,
                float* grad_directions, void* stream);

/* Standalone metadata pass, splatting/metadata.py:12-31 (_prepare). */
int gs3d_metadata(const int32_t* radii, const float* centers, const float* conics,
                  int64_t n, float* means2d, float* opacities, float* meta_conics,
                  void* stream);

/* ------------------------------------------------------------------------
 * Inclusive int32 prefix sum: primitives/tiling.py:57-64 (scan_counts,
 * wp.utils.array_scan).  total (device int64, may be NULL) receives the sum
 * computed in 64 bits; offsets overflow is reported through *total > INT32_MAX.
 * ---------------------------------------------------------------------- */
size_t gs3d_scan_scratch_bytes(int64_t n);
int gs3d_scan_i32(const int32_t* counts, int64_t n, int32_t* offsets,
                  int64_t* total, void* scratch, size_t scratch_bytes,
                  void* stream);

/* ------------------------------------------------------------------------
 * Tile-pair emission: splatting/binning.py:16-37 (duplicate, launched at
 * :192-215).  The (views*N) rows are one flat array; row r belongs to view
 * r / n and emits key ((view*tiles_per_view + y*gx + x) << 32) | bits(depth)
 * and value (r % n) at offsets[r-1] + k (row-major over its tile rectangle).
 * ---------------------------------------------------------------------- */
typedef struct gs3d_emit_args {
    int32_t n, views, width, height;
    const float* centers;     /* (views,N,2) */
    const int32_t* radii;     /* (views,N) */
    const float* depths;      /* (views,N) */
    const int32_t* offsets;   /* (views*N) inclusive scan of tiles */
    uint64_t* keys;           /* (M) */
    int32_t* values;          /* (M) */
    const float* conics;      /* (views,N,4); required unless tile_mode is GS3D_TILE_RADIUS */
    int32_t tile_mode;        /* GS3D_TILE_* (splatting/binning.py:40-68 duplicate_precise) */
} gs3d_emit_args;

size_t gs3d_emit_scratch_bytes(int64_t rows);
int gs3d_emit_keys(const gs3d_emit_args* args, void* scratch, size_t scratch_bytes,
                   void* stream);

/* ------------------------------------------------------------------------
 * Stable LSD radix sort of (uint64 key, int32 value) pairs over key bits
 * [0, end_bit): primitives/tiling.py:67-86 (sort_tile_pairs ->
 * wp.utils.radix_sort_pairs).  keys/values hold 2*count elements: the first
 * count are the input and, on return, the sorted output (the second half is
 * the ping-pong buffer, as in the reference).
 * ---------------------------------------------------------------------- */
size_t gs3d_sort_scratch_bytes(int64_t count);
int gs3d_sort_pairs_u64(uint64_t* keys, int32_t* values, int64_t count,
                        int32_t end_bit, void* scratch, size_t scratch_bytes,
                        void* stream);

/* Allocation-free variant of gs3d_sort_pairs_u64.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid allocation).
 * Same arguments and result as gs3d_sort_pairs_u64 without the scratch
 * buffer: the scratch is a static device array of GS3D_STATIC_SCRATCH_BYTES
 * per GPU (128 MiB, held until the process ends), so count is limited to
 * gs3d_sort_scratch_bytes(count) <= GS3D_STATIC_SCRATCH_BYTES (133,693,440
 * pairs); larger counts return GS3D_ERR_SCRATCH.  The stream must belong to
 * the current device.  The call allocates nothing, but every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams or
 * host threads) race and must be serialised by the caller. */
#define GS3D_STATIC_SCRATCH_BYTES (128u << 20)
int gs3d_sort_pairs_u64_static(uint64_t* keys, int32_t* values, int64_t count,
                               int32_t end_bit, void* stream);

/* Per-tile [first, last) ranges of sorted keys: primitives/tiling.py:39-54
 * (identify_ranges, launched at :87-100).  ranges (tile_count,2) must be
 * zero-initialised by the caller; tile ids >= tile_count (0xFFFFFFFF
 * included) are ignored. */
int gs3d_tile_ranges(const uint64_t* sorted_keys, int64_t count, int32_t* ranges,
                     int64_t tile_count, void* stream);

/* ------------------------------------------------------------------------
 * Grouped binning: the tile lists that splatting/binning.py:71-117 builds
 * with scan_counts, duplicate, sort_tile_pairs and identify_ranges
 * (primitives/tiling.py:39-100) -- each tile's Gaussian indices in
 * (depth bits, Gaussian index) order, tiles concatenated in global tile order
 * (view*tiles + y*gx + x), ranges [first, last) with (0, 0) for untouched
 * tiles -- built without sorting the tile pairs:
 *   1. gs3d_order_rows: stable sort of the views*N rows by the bits of their
 *      depth, giving one 64-bit record per row in that order: the row index
 *      (view*N + Gaussian) in the low 32 bits and, for tile grids of at most
 *      256 x 256 tiles, the row's tile rectangle in the high 32 bits
 *      (x0 | y0 << 8 | (x1-1) << 16 | (y1-1) << 24, 0x000000FF when culled;
 *      larger grids leave them zero).  Outside GS3D_TILE_ACCUTILE the rows
 *      that touch no tile are left out of the sort and the records end with
 *      as many fillers (row 0, rectangle 0x000000FF), which touch no group;
 *      then the inclusive scan of the number of 8x8-tile groups each record
 *      touches; two totals: group pairs (totals[0]) and tile pairs
 *      (totals[1], the reference's offsets[-1]).
 *   2. The caller reads the totals and allocates ids (tile pairs).
 *   3. gs3d_bin_rows: one (group, row) item per touched group, emitted in
 *      depth order and sorted stably by group; every group's list is cut into
 *      512-item chunks and each wavefront ranks its chunk's tiles with 64-lane
 *      ballots (one ballot per tile of the group), so every Gaussian index is
 *      written once, straight to its final position; ranges are written for
 *      every tile.
 * Limits: views*groups < 2^20, group and tile pairs < 2^31, tile grid sides
 * < 2^16.
 * ---------------------------------------------------------------------- */
typedef struct gs3d_order_args {
    int32_t n, views, width, height;
    const float* depths;      /* (views,N) */
    const float* centers;     /* (views,N,2) */
    const int32_t* radii;     /* (views,N); rows with radius <= 0 are culled */
    uint64_t* order;          /* (2*views*N): first half receives the ordered records */
    int32_t* group_offsets;   /* (views*N) inclusive scan of group counts, record order */
    int64_t* totals;          /* (2) group pairs, tile pairs */
    const float* conics;      /* (views,N,4); required unless tile_mode is GS3D_TILE_RADIUS */
    int32_t tile_mode;        /* GS3D_TILE_* */
    int32_t* tiles_out;       /* optional (views*N): every row's tile count in tile_mode */
    float* footprints;        /* ACCUTILE: (views*N,8) working footprints, 16-byte aligned, kept for gs3d_bin_rows */
    /* Bits the order sorts, 0 (all 32) or 1..32 (values below 9 sort 9):
     * the radix passes after the first take their digits from key - base,
     * base = the smallest depth key (float bits) of the rows that touch a
     * tile with its low byte cleared.  Fewer bits take fewer passes (up to
     * 26 bits: three instead of four) and order the rows correctly only if
     * every such key minus base is below 2^sort_bits, which key_bits_out
     * reports after the call: an order whose key_bits_out exceeds the bits
     * it sorted must be redone with at least that many.  Ignored (32) under
     * GS3D_TILE_ACCUTILE. */
    int32_t sort_bits;
    int32_t* key_bits_out;    /* optional (1): bit length of (largest kept key - base), 0 without kept rows; 32 for ACCUTILE */
} gs3d_order_args;

size_t gs3d_order_rows_scratch_bytes(int64_t rows);
int gs3d_order_rows(const gs3d_order_args* args, void* scratch, size_t scratch_bytes, void* stream);

typedef struct gs3d_bin_args {
    int32_t n, views, width, height;
    const float* centers;          /* (views,N,2), as given to gs3d_order_rows */
    const int32_t* radii;          /* (views,N) */
    const uint64_t* order;         /* outputs of gs3d_order_rows */
    const int32_t* group_offsets;
    int64_t group_pairs;           /* totals[0] */
    int64_t tile_pairs;            /* totals[1] */
    int32_t* ranges;               /* (views*tiles,2), every entry written */
    int32_t* ids;                  /* (tile_pairs) Gaussian index within its view */
    const float* conics;           /* (views,N,4), as given to gs3d_order_rows */
    int32_t tile_mode;             /* the tile_mode given to gs3d_order_rows */
    const float* footprints;       /* ACCUTILE: the footprints gs3d_order_rows wrote */
    /* Optional (views*tiles): per tile, the number of list entries an earlier
     * frame's forward blend read (gs3d_render_args.stop_out), negative for
     * "the whole list".  Each tile's list is then written only up to
     * stop + stop/4 + 128 entries (ranges stay whole); a forward blend given
     * the same caps reads no further and flags the tiles that needed more,
     * whose whole lists gs3d_bin_redo then writes.  NULL: whole lists. */
    const int32_t* caps;
    /* Optional, with caps: redo_list[0] is set to zero by the id-write pass
     * -- the count that the capped blend then fills (gs3d_render_args.
     * redo_list), so the caller needs no clearing of its own. */
    int32_t* redo_list;
} gs3d_bin_args;

size_t gs3d_bin_rows_scratch_bytes(int64_t group_pairs, int32_t views, int32_t width, int32_t height,
                                   int32_t tile_mode);
int gs3d_bin_rows(const gs3d_bin_args* args, void* scratch, size_t scratch_bytes, void* stream);

/* gs3d_bin_rows in two calls (radius and SnugBox modes), so that step 3's
 * first kernel can be enqueued before the caller has read the totals:
 *   gs3d_emit_group_items with args->group_pairs = a capacity C (an upper
 *   bound the caller expects, e.g. from an earlier frame) and a scratch of
 *   gs3d_bin_rows_scratch_bytes(C, ...) bytes writes the first min(totals[0], C)
 *   group items to the start of that scratch (nothing beyond C);
 *   then, once totals[0] <= C is known, gs3d_bin_emitted_rows with the true
 *   totals and the same scratch finishes the binning exactly as gs3d_bin_rows
 *   does (same ranges and ids).  When totals[0] > C the caller discards the
 *   scratch and calls gs3d_bin_rows.  ACCUTILE: GS3D_ERR_UNSUPPORTED /
 *   GS3D_ERR_ARGUMENT (its items carry tile masks; use gs3d_bin_rows).
 * Same reference counterpart as gs3d_bin_rows (splatting/binning.py:16-117). */
int gs3d_emit_group_items(const gs3d_bin_args* args, void* scratch, size_t scratch_bytes, void* stream);
int gs3d_bin_emitted_rows(const gs3d_bin_args* args, void* scratch, size_t scratch_bytes, void* stream);

/* No counterpart in the reference (the reference writes whole lists): after
 * gs3d_bin_rows / gs3d_bin_emitted_rows with caps, and with the same
 * arguments and untouched scratch, writes the whole lists of the tiles whose
 * redo flag (views*tiles int32, from gs3d_render_args.redo) is nonzero.
 * redo_list is the capped blend's gs3d_render_args.redo_list: with its count
 * zero the launch ends without reading the binning state. */
int gs3d_bin_redo(const gs3d_bin_args* args, const int32_t* redo, const int32_t* redo_list,
                  void* scratch, size_t scratch_bytes, void* stream);

/* Measurement aid, no counterpart in the reference: after gs3d_bin_rows with
 * the same arguments (caps required) and untouched scratch, writes to
 * *items_loaded (one uint64, 8-byte aligned) the number of group items the
 * capped id-write pass reads -- those of every chunk that some tile of its
 * group still needed -- without repeating the pass. */
int gs3d_bin_capped_items(const gs3d_bin_args* args, void* scratch, size_t scratch_bytes,
                          uint64_t* items_loaded, void* stream);

/* Global tile id of every listed pair: tiles[p] = t for p in ranges[t]. */
int gs3d_pair_tiles(const int32_t* ranges, int64_t tile_count, uint32_t* tiles, int64_t count,
                    void* stream);

/* keys[i] = (tiles[i] << 32) | bits(depths[view*n + ids[i]]), view =
 * tiles[i] / tiles_per_view: the reference's sorted 64-bit keys. */
int gs3d_expand_keys(const uint32_t* sorted_tiles, const int32_t* ids, int64_t count,
                     const float* depths, int32_t n, int32_t tiles_per_view,
                     uint64_t* keys, void* stream);

/* Stable LSD radix sort of (uint32 key, int32 value) pairs over key bits
 * [0, end_bit); 2*count storage as gs3d_sort_pairs_u64.  Scratch size is
 * gs3d_sort_scratch_bytes(count). */
int gs3d_sort_pairs_u32(uint32_t* keys, int32_t* values, int64_t count,
                        int32_t end_bit, void* scratch, size_t scratch_bytes,
                        void* stream);

/* ------------------------------------------------------------------------
 * Forward alpha blending on 16x16 tiles: gs3d/render.py:36-208 (render,
 * launched at :359-406).  The blended channel vector of Gaussian g in view v
 * is [features (feat_channels) | extra (extra_channels) | 1.0 if one_tail],
 * D' channels in all; background covers the feature channels only (the rest
 * are zero), as gs3d/autograd.py:41-50 builds it.
 * The blended image is written as up to three channel-last planes, the
 * layout the reference returns after its HWC split (gs3d/api.py:256-265):
 * image (views,H,W,feat_channels), image_extra (views,H,W,extra_channels)
 * and, with one_tail, image_alpha (views,H,W).
 * ---------------------------------------------------------------------- */
typedef struct gs3d_render_args {
    int32_t width, height, views;
    int32_t n;                 /* Gaussians per view (rows of centers/conics) */
    const int32_t* ranges;     /* (views*tiles,2), indices into ids */
    const int32_t* ids;        /* sorted Gaussian indices (per-view row index) */
    const float* centers;      /* (views,N,2) */
    const float* conics;       /* (views,N,4) */
    const float* features;     /* rows of feat_stride floats */
    int32_t feat_channels;
    int64_t feat_stride;       /* floats between rows */
    int64_t feat_view_stride;  /* floats between views (0 = shared) */
    const float* extra;        /* may be NULL when extra_channels == 0 */
    int32_t extra_channels;
    int64_t extra_stride, extra_view_stride;
    int32_t one_tail;          /* 1 appends the constant alpha channel */
    const float* background;   /* (views, feat_channels) rows, may be NULL */
    int64_t background_view_stride;
    float* image;              /* (views,H,W,feat_channels) */
    float* image_extra;        /* (views,H,W,extra_channels); NULL when extra_channels == 0 */
    float* image_alpha;        /* (views,H,W); NULL unless one_tail */
    float* final_t;            /* (views,H,W) */
    int32_t* contributors;     /* (views,H,W) */
    /* Optional, forward launches only: zero_count floats from zero_out
     * (16-byte aligned) are set to zero by the launch, while its blend
     * runs -- the accumulation buffers of a later gs3d_render_bwd, cleared
     * without a fill kernel of their own.  NULL / 0: nothing is cleared. */
    float* zero_out;
    int64_t zero_count;
    /* Optional, gs3d_render_fwd only -- not with statistics or pair counts
     * (no counterpart in the reference): caps as gs3d_bin_args.caps -- each tile's list is read no further than
     * the capped id-write pass wrote it.  Required with caps: redo
     * (views*tiles int32) receives 1 for the tiles that still had live
     * pixels there while their lists are longer (their outputs are then
     * incomplete), 0 for the others, and redo_list (1 + views*tiles int32,
     * redo_list[0] zero before the launch, e.g. by gs3d_bin_rows given the
     * same redo_list) receives their count in [0] and
     * the tiles from [1], in no particular order.  stop_out (views*tiles
     * int32) receives, per tile, the list entries read before every pixel
     * terminated (-1: the whole list did not suffice), the caps of a later
     * frame.  redo_pass = 1: a redo launch -- only the tiles in redo_list are
     * blended, with whole lists (after gs3d_bin_redo), into the same outputs
     * (stop_out, if given, receives their stops); caps and redo are ignored
     * and the other tiles are untouched. */
    const int32_t* caps;
    int32_t* stop_out;
    int32_t* redo;
    int32_t* redo_list;
    int32_t redo_pass;
} gs3d_render_args;

int gs3d_render_fwd(const gs3d_render_args* args, void* stream);

/* Measurement aid, no counterpart in the reference: gs3d_render_fwd (same
 * outputs) that also adds to counts[0..2] (device uint64, accumulated: the
 * caller zeroes them) the (pixel, Gaussian) pairs of the frame that the
 * reference's blend loop (gs3d/render.py:82-117) visits (list entries up to
 * and including the one that terminates the pixel, the whole list
 * otherwise), those this kernel evaluates (after strip culling, while the
 * pixel is live) and those it accepts (blends).  Used to normalise the
 * blend kernels' instruction counts. */
int gs3d_render_pair_counts(const gs3d_render_args* args, uint64_t* counts, void* stream);

/* ------------------------------------------------------------------------
 * Contribution statistics observed by the forward blend: statistics.py:16-156
 * (MaskedContributionCount, WeightedContributionSum, make_observer at
 * :46-70), fed from the accepted-blend branch of gs3d/render.py:109-115 and
 * bound at :393-397.  For each accepted blend of Gaussian g at pixel p with
 * weight alpha*T and each request r with value v = pixel_values[r][p] != 0:
 * a count request adds 1 to counts[row][g], a sum request adds v*alpha*T to
 * sums[row][g], where row numbers the requests of the same kind in order.
 * Outputs accumulate (the caller zeroes them).  Same blend outputs as
 * gs3d_render_fwd.
 * ---------------------------------------------------------------------- */
#define GS3D_MAX_STATISTICS 8
typedef struct gs3d_render_stats_args {
    int32_t requests;            /* R, 1..GS3D_MAX_STATISTICS */
    uint32_t sum_mask;           /* bit r set: request r is a weighted sum, else a masked count */
    const float* pixel_values;   /* (views, R, H*W) */
    int64_t pixel_view_stride;   /* floats between views (0 = shared) */
    int32_t* counts;             /* (views, count requests, n); NULL without count requests */
    int64_t counts_view_stride;
    float* sums;                 /* (views, sum requests, n); NULL without sum requests */
    int64_t sums_view_stride;
} gs3d_render_stats_args;

int gs3d_render_fwd_stats(const gs3d_render_args* args, const gs3d_render_stats_args* stats, void* stream);

/* ------------------------------------------------------------------------
 * Reverse traversal of the blend: gs3d/render.py:211-356 (backward, launched
 * at :409-463) with constant_tail = one_tail.  Gradients are accumulated with
 * atomics (the caller zeroes them); a wavefront reduces its 64 pixels'
 * contributions to one Gaussian before the atomic.  grad_features and
 * grad_extra honour their view strides (0 = summed over views).  Any
 * gradient pointer may be NULL except grad_centers/grad_conics.  The
 * upstream gradient arrives in the planes of the forward output, each with
 * its own pixel stride (floats between pixels, channels contiguous); a NULL
 * plane is a zero gradient.  The gradient row strides (grad_centers_stride,
 * grad_conics_stride, abs_stride, grad_feat_stride, grad_extra_stride) must
 * lie in [0, 2^31).
 * ---------------------------------------------------------------------- */
typedef struct gs3d_render_bwd_args {
    gs3d_render_args fwd;        /* same inputs; image planes unused */
    const float* upstream;       /* dL/dimage, feat_channels per pixel */
    int64_t upstream_stride;
    const float* upstream_extra; /* dL/dimage_extra, extra_channels per pixel */
    int64_t upstream_extra_stride;
    const float* upstream_alpha; /* dL/dimage_alpha, one per pixel */
    int64_t upstream_alpha_stride;
    float* grad_centers;         /* (views,N,*) rows of grad_centers_stride */
    int64_t grad_centers_stride;
    float* grad_conics;          /* (views,N,*) rows of grad_conics_stride */
    int64_t grad_conics_stride;
    float* abs_centers;          /* (views,N,*) or NULL; rows of abs_stride */
    int64_t abs_stride;
    float* grad_features;        /* rows of grad_feat_stride, view stride below */
    int64_t grad_feat_stride, grad_feat_view_stride;
    float* grad_extra;
    int64_t grad_extra_stride, grad_extra_view_stride;
} gs3d_render_bwd_args;

int gs3d_render_bwd(const gs3d_render_bwd_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GS3D_HIP_H */
