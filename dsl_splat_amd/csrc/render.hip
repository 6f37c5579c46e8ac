// Front-to-back alpha blending on 16x16 tiles and its reverse traversal.
//
// gs3d/render.py:36-208 (forward) and :211-356 (backward).  One workgroup
// per tile.  A lane owns PIX pixels of the tile (1: one pixel, 256 threads;
// 2: a horizontal pair, 128 threads; 4: a 2x2 quad, 64 threads = one
// wavefront for the whole tile).  The tile's sorted Gaussians are staged in
// LDS in batches (centre, conic + opacity, exponent cutoff and the full
// blended channel vector), so the inner loop reads only LDS broadcasts.  A
// lane leaves the inner loop once its pixels are done, a wavefront once its
// lanes are, and the workgroup stops at the next batch once all pixels are.
//
// Exponent cutoff: a Gaussian with opacity o can only reach alpha >= 1/255
// where power >= -ln(255 o); below that bound minus a 1% margin (far above
// the few-ulp error of exp, log and the product) the blend rejects the
// Gaussian without evaluating exp.  Decisions, and therefore every output,
// are identical to evaluating it.
//
// Backward: every lane accumulates its pixels' contributions to the current
// Gaussian; the wavefront sums all gradient entries together (permlane swaps
// pair the entries, a DPP row butterfly finishes them) and one atomic
// instruction adds them, one entry per lane, instead of one atomic per entry
// and pixel as in the reference.  Only batches below the largest last contributor of the
// tile are visited.
//
// Channel windows: the reference specialises its kernels on any channel count
// D' (gs3d/render.py:36-38, :211-213).  A launch here blends a window of at
// most 64 channels [c0, c0 + CH) of the D'-channel vector; wider vectors run
// one launch per window.  Forward windows are independent (the blend weights
// do not depend on the channels); window 0 writes the transmittance and last
// contributors.  Backward: the geometry launch (window 0) owns the centre,
// conic and opacity gradients, which need the dot product of the Gaussian's
// full channel vector with the pixel's upstream gradient; its window holds at
// most 64 - 8 channels, so its gradient entries fit the 64 lanes of one
// wavefront sum, and channels beyond it enter the dot product from global
// memory.  Further windows add only their channels' feature gradients.
#include "common.hpp"

#ifndef GS3D_FWD_PIX
#define GS3D_FWD_PIX 2
#endif
#ifndef GS3D_BWD_PIX
#define GS3D_BWD_PIX 2
#endif
// Pixels per lane for 9-36 channels.
#ifndef GS3D_WIDE_FWD_PIX
#define GS3D_WIDE_FWD_PIX 1
#endif
#ifndef GS3D_WIDE_BWD_PIX
#define GS3D_WIDE_BWD_PIX 1
#endif

namespace gs3d {

constexpr int kTile = 16;
constexpr int kTilePixels = kTile * kTile;

// Gaussians staged per batch.  Up to 8 channels a workgroup holds 2
// wavefronts and LDS bounds the resident workgroups: batches of 128 leave
// room for more of them (3M Gaussians, 4 x 1080p: backward 1.93 -> 1.86 ms,
// forward 1.11 -> 1.09 ms against 256; 64 and 96 were slower).  Wider
// vectors run 4 wavefronts per workgroup at one pixel per lane, where
// smaller batches only add staging rounds (32 channels: 128 was 3% slower
// than 256); the widest vectors take 128 to fit the LDS budget.
template <int CH>
struct Batch {
    static constexpr int size = CH <= 8 ? 128 : CH <= 36 ? 256 : 128;
};

// Channels of the geometry launch's window: with the 8 geometric entries
// (absolute gradients included) they fill one 64-entry wavefront sum.
constexpr int kGeomWindow = 56;
// Channels of a forward window and of a further backward window.
constexpr int kWindow = 64;

// Pixels per lane for a channel count (the widest vectors keep one pixel per
// lane to bound register use).
template <int CH, bool BWD>
struct PixFor {
    static constexpr int value = CH <= 8    ? (BWD ? GS3D_BWD_PIX : GS3D_FWD_PIX)
                                 : CH <= 36 ? (BWD ? GS3D_WIDE_BWD_PIX : GS3D_WIDE_FWD_PIX)
                                            : 1;
};

// Tile-local coordinates of pixel k of thread t.
template <int PIX>
GS3D_DEV void pixel_of(int t, int k, int& x, int& y) {
    if (PIX == 1) {
        x = t & 15;
        y = t >> 4;
    } else if (PIX == 2) {
        x = 2 * (t & 7) + k;
        y = t >> 3;
    } else {
        x = 2 * (t & 7) + (k & 1);
        y = 2 * (t >> 3) + (k >> 1);
    }
}

struct TileInfo {
    int view, x0, y0, first, last, tile;
};

// Workgroups go to the 8 XCDs in turn; within every run of 8 * GS3D_TILE_CHUNK
// workgroups, XCD x takes the x-th chunk of GS3D_TILE_CHUNK consecutive tiles
// so that neighbouring tiles, which share most of their Gaussians, meet in one
// L2 (the final partial run keeps the identity order).
#ifndef GS3D_TILE_CHUNK
#define GS3D_TILE_CHUNK 8
#endif
GS3D_DEV int tile_of_block(int b, int blocks) {
    constexpr int C = GS3D_TILE_CHUNK, R = 8 * C;
    if (C <= 1) return b;
    const int run = b / R;
    if ((run + 1) * R > blocks) return b;
    const int w = b - run * R;
    return run * R + (w & 7) * C + (w >> 3);
}

GS3D_DEV TileInfo tile_info(const gs3d_render_args& a, int tile) {
    const int gx = (a.width + kTile - 1) / kTile, gy = (a.height + kTile - 1) / kTile;
    const int per_view = gx * gy;
    TileInfo t;
    t.view = tile / per_view;
    const int local = tile - t.view * per_view;
    const int ty = local / gx, tx = local - ty * gx;
    t.x0 = tx * kTile;
    t.y0 = ty * kTile;
    t.first = a.ranges[2 * (int64_t)tile];
    t.last = a.ranges[2 * (int64_t)tile + 1];
    t.tile = tile;
    return t;
}

GS3D_DEV TileInfo tile_info(const gs3d_render_args& a) { return tile_info(a, tile_of_block(blockIdx.x, gridDim.x)); }

// Lowest power at which opacity o can still give alpha >= 1/255 (see the
// file comment); +inf rejects everything (o <= 0), -inf rejects nothing.
GS3D_DEV float power_cutoff(float o) {
    if (o > 0.0f) return -__logf(255.0f * o) - 0.01f;
    return o <= 0.0f ? __builtin_inff() : -__builtin_inff();
}

// The wavefronts of a tile each own a horizontal strip of its rows.
template <int PIX>
struct TileWaves {
    static constexpr int count = kTilePixels / PIX / 64;
    static constexpr int rows = kTile / count;
};

// Minimum over dx in [lo, hi] of Q = a dx^2 + 2 b dx dy + c dy^2 at a fixed
// dy (a > 0): Q at the clamped stationary point -b dy / a.  The reciprocal
// is approximate; moving the point by a relative 1e-7 changes Q by a second
// order amount, far inside the culling margin.
GS3D_DEV float edge_min(float a, float inv_a, float b, float c, float dy, float lo, float hi) {
    const float d = sel_clamp(-b * dy * inv_a, lo, hi);
    return (a * d + 2.0f * b * dy) * d + c * dy * dy;
}

// Bit w is set unless every pixel of wavefront w's strip is certain to reject
// the Gaussian: the ellipse {power >= cut}, its quadratic form Q widened by
// 1% + 0.01, misses the strip's rectangle of pixel centres -- first by its
// bounding box (widened by 0.01 px), then exactly: the strip is kept when
// the centre lies inside the rectangle or Q's minimum over one of the
// rectangle's four edges is within the widened bound.  Float32 evaluation of
// Q is off by at most about 8 * 2^-24 * (a + c) |d|^2, below 2e-4 Q for the
// conics culled here, and the blend's power evaluation by as little, both far
// inside the 1% margin.  Culling
// is attempted only where a*c <= 100*det (correlation below 0.995): there the
// float32 determinant is within 1.3e-5 relative of the exact one (its
// cancellation error is at most 2^-24 * 2ac <= 200 * 2^-24 * det), so the box
// stays wider than the exact ellipse's by far more than the float32 error of
// the blend's power evaluation.  More elongated conics, non-positive-definite
// ones, overflowing products and NaNs are never culled.  Rejected pairs change
// no output, so culling leaves every result identical.
template <int PIX>
GS3D_DEV uint32_t strip_mask(float2 xy, float4 con, float cut, int x0, int y0) {
    constexpr int NW = TileWaves<PIX>::count, ROWS = TileWaves<PIX>::rows;
    constexpr uint32_t all = (1u << NW) - 1u;
    const float q = -2.0f * cut;  // power >= cut  <=>  a dx^2 + 2 b dx dy + c dy^2 <= q
    if (!(q > 0.0f) && q == q) return 0u;  // nothing passes the cutoff
    const float a = con.x, b = con.y, c = con.z;
    const float ac = a * c;
    const float det = ac - b * b;
    if (!(a > 0.0f && c > 0.0f && det > 0.0f && ac < 1.0e30f && ac <= 100.0f * det && q < 1.0e30f)) return all;
    // Hardware reciprocal and square root (about one ulp each): the box is
    // widened by 1% + 0.01 px, orders of magnitude beyond their error.
    const float s = (q * 1.01f + 0.01f) * __builtin_amdgcn_rcpf(det);
    const float hx = __builtin_amdgcn_sqrtf(s * c) + 0.01f;
    const float hy = __builtin_amdgcn_sqrtf(s * a) + 0.01f;
    if (xy.x + hx < (float)x0 || xy.x - hx > (float)(x0 + kTile - 1)) return 0u;
    const float bound = q * 1.01f + 0.01f;
    const float inv_a = __builtin_amdgcn_rcpf(a), inv_c = __builtin_amdgcn_rcpf(c);
    // Centre minus pixel over the tile's columns.
    const float dx_lo = xy.x - (float)(x0 + kTile - 1), dx_hi = xy.x - (float)x0;
    uint32_t m = 0u;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const float lo = (float)(y0 + w * ROWS), hi = (float)(y0 + w * ROWS + ROWS - 1);
        if (xy.y + hy < lo || xy.y - hy > hi) continue;
        const float dy_lo = xy.y - hi, dy_hi = xy.y - lo;
        bool keep = dx_lo <= 0.0f && dx_hi >= 0.0f && dy_lo <= 0.0f && dy_hi >= 0.0f;  // centre inside
        if (!keep) {
            const float e0 = edge_min(a, inv_a, b, c, dy_lo, dx_lo, dx_hi);
            const float e1 = edge_min(a, inv_a, b, c, dy_hi, dx_lo, dx_hi);
            const float e2 = edge_min(c, inv_c, b, a, dx_lo, dy_lo, dy_hi);
            const float e3 = edge_min(c, inv_c, b, a, dx_hi, dy_lo, dy_hi);
            keep = !(sel_min(sel_min(e0, e1), sel_min(e2, e3)) > bound);
        }
        if (keep) m |= 1u << w;
    }
    return m;
}

// One staged Gaussian in LDS: conic + opacity, centre, exponent cutoff and
// the window's channels in one 16-byte-aligned record, so that the blend
// loops read all of it from one LDS address (with immediate offsets) instead
// of materialising one address per field from the scalar slot index.  The
// strip masks stay in their own array: the wavefronts read them per lane.
template <int CH>
struct alignas(16) StagedRec {
    float4 con;
    float2 xy;
    float cut;
    float pad;
    float f[CH];
};

// Stage one Gaussian's centre, conic, cutoff, strip mask and the channels
// [c0, c0 + CH) of its channel vector (zero beyond D').
template <int CH, int PIX, bool LAUNDER = false>
GS3D_DEV void stage_gaussian(const gs3d_render_args& a, const TileInfo& t, int32_t g, int slot, int c0,
                             StagedRec<CH>* s_g, uint32_t* s_mask) {
    const int view = t.view;
    const int64_t row = (int64_t)view * a.n + g;
    const float2 xy = reinterpret_cast<const float2*>(a.centers)[row];
    const float4 con = reinterpret_cast<const float4*>(a.conics)[row];
    // The channel vector [features | extra | 1]: its loads are issued with
    // the centre's and conic's, before the cutoff and strip mask wait for
    // those (compile-time channel slots, predicated on the counts).
    const int F = a.feat_channels, E = a.extra_channels;
    const float* f = a.features + view * a.feat_view_stride + (int64_t)g * a.feat_stride;
    const float* e = E > 0 ? a.extra + view * a.extra_view_stride + (int64_t)g * a.extra_stride : nullptr;
    float v[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int gc = c0 + c;
        float x = 0.0f;
        if (gc < F)
            x = f[gc];
        else if (gc < F + E)
            x = e[gc - F];
        else if (gc == F + E && a.one_tail)
            x = 1.0f;
        v[c] = x;
    }
    StagedRec<CH>& rec = s_g[slot];
    rec.con = con;
    rec.xy = xy;
    const float cut = power_cutoff(con.w);
    rec.cut = cut;
    int x0 = t.x0, y0 = t.y0;
    if constexpr (LAUNDER) {
        // The tile origin passes through an opaque scalar move, so that the
        // strip edges' float conversions are redone here (a few VALU per
        // staged Gaussian) instead of being hoisted out of the batch loop
        // into VGPRs that stay live over the whole traversal.
        asm volatile("" : "+s"(x0), "+s"(y0));
    }
    s_mask[slot] = strip_mask<PIX>(xy, con, cut, x0, y0);
#pragma unroll
    for (int c = 0; c < CH; ++c) rec.f[c] = v[c];
}

// 0.0f that the compiler cannot see through (a register written by an
// opaque move), so accumulators initialised from it are updated in place.
GS3D_DEV float opaque_zero() {
    float z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    return z;
}

// Two opaque zeros from one 64-bit move.
GS3D_DEV void opaque_zero2(float& a, float& b) {
    uint64_t z;
    asm volatile("v_mov_b64 %0, 0" : "=v"(z));
    a = __uint_as_float((uint32_t)z);
    b = __uint_as_float((uint32_t)(z >> 32));
}

// One staged Gaussian as the blend loops read it from LDS.  The loops load
// the next Gaussian of their wavefront before blending the current one, so
// the LDS latency overlaps the arithmetic.
template <int CH>
struct Staged {
    float2 xy;
    float4 con;
    float cut;
    float f[CH];
};

template <int CH>
GS3D_DEV Staged<CH> load_staged(int j, const StagedRec<CH>* s_g) {
    const StagedRec<CH>& rec = s_g[j];
    Staged<CH> g;
    g.xy = rec.xy;
    g.con = rec.con;
    g.cut = rec.cut;
#pragma unroll
    for (int c = 0; c < CH; ++c) g.f[c] = rec.f[c];
    return g;
}

// Contribution statistics of one accepted Gaussian (statistics.py:46-70,
// observed at gs3d/render.py:109-115).  Each lane forms, for every request r
// of the launch (RB, the request count rounded up to 1, 2, 4 or 8), its
// pixels' part: the number of accepted pixels whose value is nonzero for a
// masked count, the sum of value * alpha * T over them for a weighted sum.
// A count request's pixel values are replaced by 0/1 masks when they are
// loaded, so both kinds are one multiply-add per pixel: value times
// (accepted ? alpha * T : 0) for a sum, mask times (accepted ? 1 : 0) for a
// count.  That product form is exact only for finite values (a rejected
// pixel's value times zero), so a wavefront with a non-finite value selects
// each term instead (wave-uniform choice).  One wavefront sum covers all
// requests together (permlane pairing and a DPP row butterfly, as in the
// backward), and each lane that holds a request's total (stat_lane) adds it
// to the Gaussian's LDS slot, where the tile's wavefronts meet; once every
// wavefront is past the batch, the thread that staged the Gaussian adds the
// slot's nonzero totals to the request rows with one global atomic each
// (flush_statistics): half the global atomics of one per wavefront.
// Counts are exact (at most 256 per tile, summed in float32 without
// rounding); sums differ from per-pixel atomics only in the order of the
// float additions, which atomics leave unspecified anyway.
template <int RB>
GS3D_DEV int stat_lane(const gs3d_render_stats_args& st, int lane) {
    int r = 0;
    if constexpr (RB == 1) {
        if (lane != 63) return -1;
    } else {
        constexpr int rows = (RB + 3) / 4;
        r = wave_sum_rows_value(lane);
        if ((lane & 15) >= rows || r >= RB) return -1;
    }
    return r < st.requests ? r : -1;
}

// Adds a staged Gaussian's per-request totals (slot[r]) to the request rows
// of view `view` (each row among the rows of its kind) and clears the slot.
template <int RB>
GS3D_DEV void flush_statistics(const gs3d_render_stats_args& st, int view, int n, int32_t g, float* slot) {
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        if (r >= st.requests) break;
        const float v = slot[r];
        slot[r] = 0.0f;
        if (v == 0.0f) continue;
        const uint32_t before = st.sum_mask & ((1u << r) - 1u);
        if ((st.sum_mask >> r) & 1u)
            atomicAdd(st.sums + view * st.sums_view_stride + (int64_t)__builtin_popcount(before) * n + g, v);
        else
            atomicAdd(st.counts + view * st.counts_view_stride + (int64_t)(r - __builtin_popcount(before)) * n + g,
                      (int)v);
    }
}

// KINDS: the requests' kinds as a compile-time sum mask (bit r set: request
// r is a weighted sum) for launches of one or two requests, -1 to read them
// from st.sum_mask.
template <int PIX, int RB, int KINDS>
GS3D_DEV void observe_statistics(const gs3d_render_stats_args& st, int dst_r, float* slot,
                                 const bool (&acc)[PIX], const float (&w)[PIX], const float (&val)[PIX][RB],
                                 bool finite, int lane) {
    float e[RB];
    if (finite) {
        float one[PIX];
#pragma unroll
        for (int k = 0; k < PIX; ++k) one[k] = acc[k] ? 1.0f : 0.0f;
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            // wave-uniform; a compile-time constant for KINDS >= 0
            const bool is_sum = KINDS >= 0 ? ((KINDS >> r) & 1) != 0 : ((st.sum_mask >> r) & 1u) != 0;
            float v = 0.0f;
#pragma unroll
            for (int k = 0; k < PIX; ++k) v = __builtin_fmaf(val[k][r], is_sum ? w[k] : one[k], v);
            e[r] = v;
        }
    } else {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const bool is_sum = (st.sum_mask >> r) & 1u;
            float v = 0.0f;
#pragma unroll
            for (int k = 0; k < PIX; ++k) {
                const bool hit = acc[k] && val[k][r] != 0.0f;
                v += hit ? (is_sum ? val[k][r] * w[k] : 1.0f) : 0.0f;
            }
            e[r] = v;
        }
    }
    float total;
    if constexpr (RB == 1) {
        total = wave_sum_to_lane63(e[0]);
    } else {
        constexpr int rows = (RB + 3) / 4;
        float sums[rows];
        wave_sum_rows<RB>(e, sums);
#pragma unroll
        for (int q = 0; q < rows; ++q) asm volatile("" : "+v"(sums[q]));
        total = sums[0];
#pragma unroll
        for (int q = 1; q < rows; ++q) total = ((lane & 15) == q) ? sums[q] : total;
    }
    if (dst_r >= 0 && total != 0.0f) atomicAdd(slot + dst_r, total);  // LDS
}

// Up to 8 channels the kernel is held to 80 VGPRs (6 wavefronts per SIMD
// instead of 5: 1.180 -> 1.130 ms on RGB); wider channel vectors keep the
// registers they need.
//
// MODE: 0 plain; 1 with contribution statistics; 2 also counting (pixel,
// Gaussian) pairs into counts[0..2]: visited as the reference's loop visits
// them (list entries up to and including the one that terminates the pixel,
// the whole list otherwise), evaluated by this kernel (after strip culling,
// while the pixel is live) and accepted (blended).
//
// RB: statistics requests compiled in (MODE 1; the launch's request count
// rounded up to 1, 2, 4 or 8), so that only their pixel values take
// registers; KINDS: their kinds as a sum mask for one or two requests (the
// observer then needs no per-request selects), -1 otherwise.
//
// LISTS (MODE 0): 0 whole lists; 1 lists capped by gs3d_render_args.caps
// and/or stops reported (stop_out, redo flags); 2 a redo launch
// (gs3d_render_args.redo_pass), whose workgroups walk the tiles listed by the
// capped launch.  Only the instantiations that use them carry the stop
// tracking and the loop.
template <int CH, int PIX, int MODE, int RB = 1, int KINDS = -1, int LISTS = 0>
__global__ __launch_bounds__(kTilePixels / PIX) __attribute__((amdgpu_waves_per_eu(CH <= 4 ? 6 : CH <= 8 ? 5 : 1))) void render_fwd_kernel(gs3d_render_args a, gs3d_render_stats_args st, int c0, unsigned long long* counts) {
    constexpr bool STATS = MODE == 1, COUNTS = MODE == 2;
    constexpr int NT = kTilePixels / PIX;
    constexpr int B = Batch<CH>::size;
    __shared__ StagedRec<CH> s_g[B];
    __shared__ uint32_t s_mask[B];
    // Per staged Gaussian: the tile's totals of every statistics request.
    __shared__ float s_stat[STATS ? B * RB : 1];
    static_assert(LISTS == 0 || MODE == 0, "capped lists neither count pairs nor total statistics");
    // The blend of one tile: a normal launch blends the tile of its
    // workgroup, a redo launch walks the tiles that the capped launch listed.
    auto blend = [&](const TileInfo t) {
        // With caps the tile's list is read up to list_cap of its previous stop
        // (the id-write pass wrote that far); a redo reads whole lists.
        int last = t.last;
        bool capped = false;
        if constexpr (LISTS == 1) {
            if (a.caps) {
                const uint32_t cap = list_cap(a.caps[t.tile]);
                if ((uint32_t)(t.last - t.first) > cap) {
                    last = t.first + (int)cap;
                    capped = true;
                }
            }
        }
        const int D = a.feat_channels + a.extra_channels + (a.one_tail ? 1 : 0);
        const int lane = lane_id(), wave = threadIdx.x >> 6;
        if constexpr (STATS)
            for (int e = threadIdx.x; e < B * RB; e += NT) s_stat[e] = 0.0f;
        if (c0 == 0 && a.zero_out) {
            // The blend VJP's accumulation buffers, cleared by the first
            // window's launch: the stores drain while the blend computes.
            typedef float zero4 __attribute__((ext_vector_type(4)));
            const int64_t n4 = a.zero_count >> 2;
            zero4* z = reinterpret_cast<zero4*>(a.zero_out);
            const int64_t step = (int64_t)gridDim.x * NT;
            for (int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x; i < n4; i += step)
                __builtin_nontemporal_store(zero4{0.0f, 0.0f, 0.0f, 0.0f}, z + i);
            if (blockIdx.x == 0 && threadIdx.x < (a.zero_count & 3)) a.zero_out[(n4 << 2) + threadIdx.x] = 0.0f;
        }
        float fx[PIX], fy[PIX], T[PIX], color[PIX][CH];
        int px[PIX], py[PIX], last_contributor[PIX];
        bool done[PIX];
        float val[PIX][STATS ? RB : 1];
        int visited[PIX];
        uint32_t evaluated = 0, accepted = 0;
#pragma unroll
        for (int k = 0; k < PIX; ++k) {
            int lx, ly;
            pixel_of<PIX>(threadIdx.x, k, lx, ly);
            px[k] = t.x0 + lx;
            py[k] = t.y0 + ly;
            fx[k] = (float)px[k];
            fy[k] = (float)py[k];
            done[k] = !(px[k] < a.width && py[k] < a.height);
            visited[k] = done[k] ? 0 : last - t.first;  // the whole list unless the pixel terminates
            T[k] = 1.0f;
            last_contributor[k] = 0;
#pragma unroll
            for (int c = 0; c < CH; ++c) color[k][c] = 0.0f;
            if constexpr (STATS) {
                const float* pv = st.pixel_values + t.view * st.pixel_view_stride + (int64_t)py[k] * a.width + px[k];
                const int64_t plane = (int64_t)a.width * a.height;
#pragma unroll
                for (int r = 0; r < RB; ++r) {
                    const float v = (r < st.requests && !done[k]) ? pv[r * plane] : 0.0f;
                    // Count requests keep a 0/1 mask (see observe_statistics).
                    val[k][r] = ((st.sum_mask >> r) & 1u) ? v : (v != 0.0f ? 1.0f : 0.0f);
                }
            }
        }
        // Each thread stages at most one Gaussian per batch (B <= NT); its index
        // for the next batch is loaded while the current batch blends (clamped
        // into the list, so the load is unconditional).
        static_assert(B <= NT, "one staged Gaussian per thread and batch");
        int32_t next_id = last > t.first ? a.ids[min(t.first + (int)threadIdx.x, last - 1)] : 0;
        int stat_r = -1;
        bool stat_finite = true;
        // The Gaussian this thread staged for the batch being blended, whose
        // statistics slot it flushes (-1: none).
        int32_t flush_id = -1;
        auto flush = [&]() {
            if constexpr (STATS) {
                if (flush_id >= 0) flush_statistics<RB>(st, t.view, a.n, flush_id, &s_stat[threadIdx.x * RB]);
                flush_id = -1;
            }
        };
        if constexpr (STATS) {
            stat_r = stat_lane<RB>(st, lane);
            bool finite = true;
#pragma unroll
            for (int k = 0; k < PIX; ++k)
#pragma unroll
                for (int r = 0; r < RB; ++r) finite = finite && __builtin_fabsf(val[k][r]) <= 3.0e38f;
            stat_finite = __ballot(!finite) == 0;
        }
        int stop = -1;  // list entries read before every pixel terminated (-1: never)
        for (int begin = t.first; begin < last; begin += B) {
            bool active = false;
#pragma unroll
            for (int k = 0; k < PIX; ++k) active = active || !done[k];
            const int active_threads = __syncthreads_count(active);
            flush();  // every wavefront is past the previous batch
            if (active_threads == 0) {
                stop = begin - t.first;
                break;
            }
            if (threadIdx.x < B) {
                const int e = threadIdx.x;
                const int32_t g = next_id;
                if (begin + e < last) {
                    // The 4-channel plain blend fits its registers without the
                    // tile-origin laundering (and is fastest so).
                    stage_gaussian<CH, PIX, (STATS || CH > 4)>(a, t, g, e, c0, s_g, s_mask);
                    if constexpr (STATS) flush_id = g;
                }
                if (begin + B < last) next_id = a.ids[min(begin + B + e, last - 1)];
            }
            __syncthreads();
            const int cnt = min(B, last - begin);
            bool live = true;
            for (int c0 = 0; c0 < cnt && live; c0 += 64) {
                // This wavefront's Gaussians of the next 64, in list order.
                uint64_t todo = __ballot(c0 + lane < cnt && ((s_mask[min(c0 + lane, B - 1)] >> wave) & 1u));
                if (!todo) continue;
                // Blend one Gaussian (batch slot j) into this lane's pixels.
                auto blend = [&](const Staged<CH>& g, int j) {
                    const int contributor = begin - t.first + j + 1;  // list position, 1-based
                    bool acc[PIX];
                    float wk[PIX];
                    // Branch-free per pixel except for the exponential: a
                    // divergent branch per test costs more in exec-mask work than
                    // the selects it replaces (the wavefront issues the tail
                    // whenever any lane needs it).  Updates are selected, not
                    // multiplied by zero, so non-finite features of a rejected
                    // Gaussian cannot reach the pixel.
#pragma unroll
                    for (int k = 0; k < PIX; ++k) {
                        const float dx = g.xy.x - fx[k], dy = g.xy.y - fy[k];
                        const float power = blend_power(g.con.x, g.con.y, g.con.z, dx, dy);
                        if constexpr (COUNTS) evaluated += done[k] ? 0u : 1u;
                        const bool in = !done[k] && power <= 0.0f && power >= g.cut;
                        float e = 0.0f;
                        if (in) e = blend_exp(power);
                        const float alpha = in ? sel_min(0.99f, g.con.w * e) : 0.0f;
                        const bool take = alpha >= 1.0f / 255.0f;
                        const float next_t = T[k] * (1.0f - alpha);
                        const bool term = take && next_t < 0.0001f;
                        const bool upd = take && !term;
                        if constexpr (COUNTS) {
                            visited[k] = term ? contributor : visited[k];
                            accepted += upd ? 1u : 0u;
                        }
                        done[k] = done[k] || term;
                        const float w = alpha * T[k];
#pragma unroll
                        for (int c = 0; c < CH; ++c) {
                            const float nc = __builtin_fmaf(g.f[c], w, color[k][c]);
                            color[k][c] = upd ? nc : color[k][c];
                        }
                        T[k] = upd ? next_t : T[k];
                        last_contributor[k] = upd ? contributor : last_contributor[k];
                        acc[k] = upd;
                        wk[k] = upd ? w : 0.0f;
                    }

                    if constexpr (STATS) {
                        bool hit = false;
#pragma unroll
                        for (int k = 0; k < PIX; ++k) hit = hit || acc[k];
                        if (__ballot(hit))
                            observe_statistics<PIX, RB, KINDS>(st, stat_r, &s_stat[j * RB], acc, wk, val, stat_finite, lane);
                    }
                };
                auto alive = [&]() {
                    bool any = false;
#pragma unroll
                    for (int k = 0; k < PIX; ++k) any = any || !done[k];
                    return __ballot(any) != 0;
                };
                auto take = [&]() {
                    const int j = c0 + __builtin_ctzll(todo);
                    todo &= todo - 1;
                    return j;
                };
                if constexpr ((STATS && (RB > 2 || CH > 4)) || (CH > 16 && CH <= 36)) {
                    // Loads at use: the pipelined form's extra registers would
                    // cost occupancy -- with statistics beyond two requests (their
                    // pixel values take 4 * PIX registers or more) or four
                    // channels (up to both, the pipelined form fits 80 VGPRs),
                    // and for 36
                    // channels a third wavefront per SIMD (148 VGPRs against 190
                    // with the next Gaussian's vector prefetched: 0.83 -> 0.72
                    // ms on the 32-feature workload).
                    while (todo) {
                        if (!alive()) {
                            live = false;
                            break;
                        }
                        const int j = take();
                        blend(load_staged<CH>(j, s_g), j);
                    }
                } else {
                    // Unrolled by two: the next Gaussian is loaded into the other
                    // buffer before the current one is blended.
                    int ja = take(), jb = 0;
                    Staged<CH> ga = load_staged<CH>(ja, s_g), gb;
                    while (true) {
                        if (!alive()) {
                            live = false;
                            break;
                        }
                        bool more = todo != 0;
                        if (more) {
                            jb = take();
                            gb = load_staged<CH>(jb, s_g);
                        }
                        blend(ga, ja);
                        if (!more) break;
                        // Liveness is checked once per two Gaussians: a Gaussian
                        // blended after every pixel is done changes nothing (no
                        // pixel accepts it), and the check costs VALU and scalar
                        // work on every Gaussian (1091 -> 1067 us for the
                        // 3M-Gaussian forward blend).
                        more = todo != 0;
                        if (more) {
                            ja = take();
                            ga = load_staged<CH>(ja, s_g);
                        }
                        blend(gb, jb);
                        if (!more) break;
                    }
                }
            }
        }
        if constexpr (STATS) {
            // The last batch, when the loop ran to the end of the list.
            __syncthreads();
            flush();
        }
        if constexpr (LISTS != 0) {
            if (stop < 0) {
                // The loop ran to the end of the list it had: all of it read.
                bool active = false;
#pragma unroll
                for (int k = 0; k < PIX; ++k) active = active || !done[k];
                if (__syncthreads_count(active) == 0) stop = last - t.first;
            }
            if (threadIdx.x == 0 && c0 == 0) {
                // A capped tile with pixels still live needs its whole list:
                // flagged and listed for a redo (its outputs here are
                // incomplete).
                if (LISTS == 1 && a.redo) {
                    const bool redo = capped && stop < 0;
                    a.redo[t.tile] = redo ? 1 : 0;
                    if (redo) {
                        // The list holds one slot per tile (a count left
                        // uncleared cannot send the store out of it).
                        const int slot = atomicAdd(a.redo_list, 1);
                        if ((unsigned)slot < (unsigned)gridDim.x) a.redo_list[1 + slot] = t.tile;
                    }
                }
                if (a.stop_out) a.stop_out[t.tile] = stop;
            }
        }
        const float* bg = a.background ? a.background + t.view * a.background_view_stride : nullptr;
        const int F = a.feat_channels, E = a.extra_channels;
#pragma unroll
        for (int k = 0; k < PIX; ++k) {
            if (!(px[k] < a.width && py[k] < a.height)) continue;
            const int64_t pix = ((int64_t)t.view * a.height + py[k]) * a.width + px[k];
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int gc = c0 + c;
                if (gc >= D) continue;
                const float v = __builtin_fmaf(T[k], (bg && gc < F) ? bg[gc] : 0.0f, color[k][c]);
                if (gc < F)
                    a.image[pix * F + gc] = v;
                else if (gc < F + E)
                    a.image_extra[pix * E + (gc - F)] = v;
                else
                    a.image_alpha[pix] = v;
            }
            if (c0 == 0) {
                a.final_t[pix] = T[k];
                a.contributors[pix] = last_contributor[k];
            }
        }
        if constexpr (COUNTS) {
            uint64_t v = 0;
#pragma unroll
            for (int k = 0; k < PIX; ++k) v += (uint64_t)visited[k];
            uint64_t e = evaluated, c = accepted;
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) {
                v += (uint64_t)__shfl_xor((long long)v, d, 64);
                e += (uint64_t)__shfl_xor((long long)e, d, 64);
                c += (uint64_t)__shfl_xor((long long)c, d, 64);
            }
            if (lane == 0) {
                atomicAdd(counts, (unsigned long long)v);
                atomicAdd(counts + 1, (unsigned long long)e);
                atomicAdd(counts + 2, (unsigned long long)c);
            }
        }
    };
    if constexpr (LISTS == 2) {
        // redo_list[0] tiles from redo_list[1], over a grid smaller than the
        // frame's; the next tile reuses the staging LDS.  Counts and tile
        // indices beyond the frame's tiles are ignored.
        const int tiles = a.views * ((a.width + kTile - 1) / kTile) * ((a.height + kTile - 1) / kTile);
        const int items = min(a.redo_list[0], tiles);
        for (int item = blockIdx.x; item < items; item += gridDim.x) {
            const int tile = a.redo_list[1 + item];
            if ((unsigned)tile >= (unsigned)tiles) continue;  // uniform: one value per workgroup
            blend(tile_info(a, tile));
            __syncthreads();
        }
    } else {
        blend(tile_info(a));
    }
}

// Channels [c_begin, D) of Gaussian g's vector dotted with the upstream
// gradient of pixel (px, py) (geometry launch of a vector wider than its
// window: the channels beyond the window come from global memory).
GS3D_DEV float rest_dot(const gs3d_render_bwd_args& b, int view, int64_t g, float px, float py, int c_begin) {
    const gs3d_render_args& a = b.fwd;
    const int64_t pix = ((int64_t)view * a.height + (int)py) * a.width + (int)px;
    const int F = a.feat_channels, E = a.extra_channels;
    float dot = 0.0f;
    int c = c_begin;
    if (c < F) {
        const float* f = a.features + view * a.feat_view_stride + g * a.feat_stride;
        const float* u = b.upstream ? b.upstream + pix * b.upstream_stride : nullptr;
        for (; c < F; ++c) dot = __builtin_fmaf(f[c], u ? u[c] : 0.0f, dot);
    }
    if (c < F + E) {
        const float* f = a.extra + view * a.extra_view_stride + g * a.extra_stride;
        const float* u = b.upstream_extra ? b.upstream_extra + pix * b.upstream_extra_stride : nullptr;
        for (; c < F + E; ++c) dot = __builtin_fmaf(f[c - F], u ? u[c - F] : 0.0f, dot);
    }
    if (c == F + E && a.one_tail && b.upstream_alpha) dot += b.upstream_alpha[pix * b.upstream_alpha_stride];
    return dot;
}

// Four channels fit 80 VGPRs, six wavefronts per SIMD (the LDS limit of a
// 13 KiB block); with absolute gradients the uncapped allocation is 83.
//
// GEOM: the geometry launch (window 0, c0 = 0): centre, conic and opacity
// gradients (+ absolute centre gradients with ABS) and the window's feature
// gradients; channels from CH on, if any, enter the alpha gradient through
// rest_dot.  !GEOM: a further window [c0, c0 + CH), feature gradients only.
template <int CH, bool ABS, int PIX, bool GEOM>
__global__ __launch_bounds__(kTilePixels / PIX) __attribute__((amdgpu_waves_per_eu(CH <= 4 ? 6 : 1))) void render_bwd_kernel(gs3d_render_bwd_args b, int c0) {
    constexpr int NT = kTilePixels / PIX;
    constexpr int B = Batch<CH>::size;
    // Gradient entries per Gaussian: [centre xy, conic abc, opacity, |centre| xy]
    // for the geometry launch, then the window's channels; one wavefront sum
    // covers at most 64.
    constexpr int FB = GEOM ? (ABS ? 8 : 6) : 0;
    constexpr int NV = FB + CH;
    static_assert(NV <= 64, "one wavefront sum holds at most 64 gradient entries");
    constexpr int R = (NV + 3) / 4;
    __shared__ StagedRec<CH> s_g[B];
    __shared__ uint32_t s_mask[B];
    __shared__ int32_t s_id[B];
    __shared__ int s_max_last;
    const gs3d_render_args& a = b.fwd;
    const TileInfo t = tile_info(a);
    const int D = a.feat_channels + a.extra_channels + (a.one_tail ? 1 : 0);
    const int Dg = D - (a.one_tail ? 1 : 0);
    // Only the widest geometry window can be followed by further channels.
    const bool rest = GEOM && CH == kGeomWindow && D > CH;  // wave-uniform
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    // Per pixel: S = sum_c accum_c * grad_c, the colour accumulated behind
    // the current Gaussian dotted with the upstream gradient.  With
    // dot = sum_c f_c * grad_c the alpha gradient sum_c (f_c - accum_c) grad_c
    // (gs3d/render.py:300-312) is E = dot - S, and
    // accum_c = la last_c + (1 - la) accum_c becomes S = S + la E_last with
    // la and E_last those of the last accepted Gaussian: no per-channel state
    // besides grad.  bg_t = -T_final * sum_c bg_c grad_c is the background
    // term, divided by the transmittance factors as they are undone.
    float fx[PIX], fy[PIX], T[PIX], bg_t[PIX], last_alpha[PIX], S[PIX], last_e[PIX];
    float grad[PIX][CH];
    int last_contributor[PIX];
    bool inside[PIX];
    if (threadIdx.x == 0) s_max_last = 0;
    const float* bg = a.background ? a.background + t.view * a.background_view_stride : nullptr;
    int my_max = 0;
    // Per-pixel inputs: every load first, from the pixel clamped into the
    // image (the branches below depend only on the channel, so all lanes
    // load together), then the pixels outside the image are cleared.  A load
    // under a per-lane condition would be a branch that waits for its data.
    const int F = a.feat_channels, E = a.extra_channels;
    int64_t pix[PIX];
#pragma unroll
    for (int k = 0; k < PIX; ++k) {
        int lx, ly;
        pixel_of<PIX>(threadIdx.x, k, lx, ly);
        const int x = t.x0 + lx, y = t.y0 + ly;
        fx[k] = (float)x;
        fy[k] = (float)y;
        inside[k] = x < a.width && y < a.height;
        pix[k] = ((int64_t)t.view * a.height + min(y, a.height - 1)) * a.width + min(x, a.width - 1);
        T[k] = a.final_t[pix[k]];
        last_contributor[k] = a.contributors[pix[k]];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            // The channel's source (wave-uniform selects, no branch); channels
            // without one read final_t and take 0.
            const int gc = c0 + c;
            const float* src = gc < F ? b.upstream : gc < F + E ? b.upstream_extra : b.upstream_alpha;
            const int64_t stride = gc < F ? b.upstream_stride
                                          : gc < F + E ? b.upstream_extra_stride : b.upstream_alpha_stride;
            const int off = gc < F ? gc : gc < F + E ? gc - F : 0;
            const bool has = gc < D && src != nullptr;
            const float u = has ? src[pix[k] * stride + off] : a.final_t[pix[k]];
            grad[k][c] = has ? u : 0.0f;
        }
    }
#pragma unroll
    for (int k = 0; k < PIX; ++k) {
        bg_t[k] = last_alpha[k] = S[k] = last_e[k] = 0.0f;
        if (!inside[k]) {
            T[k] = 0.0f;
            last_contributor[k] = 0;
#pragma unroll
            for (int c = 0; c < CH; ++c) grad[k][c] = 0.0f;
            continue;
        }
        if (GEOM) {
            float bg_grad = 0.0f;
            if (bg) {
#pragma unroll
                for (int c = 0; c < CH; ++c) {
                    const int gc = c0 + c;
                    bg_grad += (gc < D && gc < F ? bg[gc] : 0.0f) * grad[k][c];
                }
                // Background channels beyond the window.
                if (b.upstream)
                    for (int gc = CH; gc < F; ++gc) bg_grad += bg[gc] * b.upstream[pix[k] * b.upstream_stride + gc];
            }
            bg_t[k] = -T[k] * bg_grad;
        }
        my_max = max(my_max, last_contributor[k]);
    }
    __syncthreads();
    if (my_max > 0) atomicMax(&s_max_last, my_max);
    __syncthreads();
    const int max_last = min(s_max_last, t.last - t.first);
    // Gradient entry this lane adds after the wavefront sums (see
    // wave_sum_rows): entry k of Gaussian g lives at dst_base + g * dst_step.
    float* dst_base = nullptr;
    uint32_t dst_step = 0;  // row strides below 2^31 (checked on the host)
    float dst_scale = 1.0f;
    {
        const int k = wave_sum_rows_value(lane);
        if (GEOM) {
            if (k < 2 || k == 3) dst_scale = -1.0f;
            if (k == 2 || k == 4) dst_scale = -0.5f;
        }
        const int64_t row0 = (int64_t)t.view * a.n;
        if ((lane & 15) >= R || k >= NV) {
        } else if (GEOM && k < 2) {
            dst_base = b.grad_centers + row0 * b.grad_centers_stride + k;
            dst_step = b.grad_centers_stride;
        } else if (GEOM && k < 6) {
            dst_base = b.grad_conics + row0 * b.grad_conics_stride + (k - 2);
            dst_step = b.grad_conics_stride;
        } else if (GEOM && ABS && k < 8) {
            dst_base = b.abs_centers + row0 * b.abs_stride + (k - 6);
            dst_step = b.abs_stride;
        } else {
            const int c = c0 + k - FB;
            if (c < a.feat_channels) {
                if (b.grad_features) {
                    dst_base = b.grad_features + t.view * b.grad_feat_view_stride + c;
                    dst_step = b.grad_feat_stride;
                }
            } else if (c < Dg && b.grad_extra) {
                dst_base = b.grad_extra + t.view * b.grad_extra_view_stride + (c - a.feat_channels);
                dst_step = b.grad_extra_stride;
            }
        }
    }
    // Largest last contributor among this wavefront's pixels (wave-uniform).
    const int lane_last = my_max;
    int wave_last = my_max;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) wave_last = max(wave_last, __shfl_xor(wave_last, d, 64));
    // As in the forward: one staged Gaussian per thread and batch, its index
    // for the next batch loaded while the current one is traversed.
    static_assert(B <= NT, "one staged Gaussian per thread and batch");
    int32_t next_id = max_last > 0 ? a.ids[t.first + max(max_last - 1 - (int)threadIdx.x, 0)] : 0;
    for (int top = max_last; top > 0; top -= B) {
        __syncthreads();
        if (threadIdx.x < B) {
            const int e = threadIdx.x;
            const int p = top - 1 - e;
            const int32_t g = next_id;
            if (p >= 0) {
                s_id[e] = g;
                // Tile origin laundered (see stage_gaussian): 75 instead of
                // 79 VGPRs, no spill with absolute gradients, 1.7% faster
                // at 36 channels.
                stage_gaussian<CH, PIX, true>(a, t, g, e, c0, s_g, s_mask);
            }
            if (top > B) next_id = a.ids[t.first + max(p - B, 0)];
        }
        __syncthreads();
        const int cnt = min(B, top);
        for (int c0b = 0; c0b < cnt; c0b += 64) {
          // This wavefront's Gaussians of the next 64 that lie before its
          // pixels' last contributors, in traversal order.
          const int e = c0b + lane;
          uint64_t todo = __ballot(e < cnt && top - 1 - e < wave_last && ((s_mask[min(e, B - 1)] >> wave) & 1u));
          while (todo) {
            const int j = c0b + __builtin_ctzll(todo);
            todo &= todo - 1;
            const int pos = top - 1 - j;
            // Pixels outside the image have last contributor 0.
            if (__ballot(pos < lane_last) == 0) continue;
            const float2 xy = s_g[j].xy;
            const float4 con = s_g[j].con;
            const float cut = s_g[j].cut;
            const float* f = s_g[j].f;
            // Accumulators start from an opaque zero: a literal zero would be
            // folded into each accumulator's first FMA, and every path that
            // skips a pixel would then re-materialise the zeros.  vals holds,
            // in gradient-entry order, sum w (a dx + b dy), sum w (c dy + b dx),
            // sum w dx dx, sum w dx dy, sum w dy dy with w = o G dL/dalpha,
            // then sum G dL/dalpha, the absolute centre terms and the feature
            // terms; the constant factors (-1, -1/2) are applied per lane
            // after the wavefront sum.
            float vals[NV];
#pragma unroll
            for (int i = 0; i + 1 < NV; i += 2) opaque_zero2(vals[i], vals[i + 1]);
            if constexpr (NV % 2) vals[NV - 1] = opaque_zero();
            bool accepted = false;
#pragma unroll
            for (int k = 0; k < PIX; ++k) {
                if (!(pos < last_contributor[k])) continue;
                const float dx = xy.x - fx[k], dy = xy.y - fy[k];
                const float power = blend_power(con.x, con.y, con.z, dx, dy);
                if (!(power <= 0.0f) || !(power >= cut)) continue;
                const float G = blend_exp(power);
                const float og = con.w * G;
                const float alpha = sel_min(0.99f, og);
                if (!(alpha >= 1.0f / 255.0f)) continue;
                accepted = true;
                // Gradients only need tolerance-level agreement: one hardware
                // reciprocal (1 - alpha >= 0.01) and fused multiply-adds.
                const float inv = __builtin_amdgcn_rcpf(1.0f - alpha);
                T[k] = T[k] * inv;
                const float aT = alpha * T[k];
                // Every compiled channel slot is processed: slots at or beyond
                // D hold zero features and zero upstream gradients (no
                // contribution), and the constant alpha channel's entry has no
                // destination, so no per-channel branch is needed.
#pragma unroll
                for (int c = 0; c < CH; ++c) vals[FB + c] = __builtin_fmaf(aT, grad[k][c], vals[FB + c]);
                if constexpr (GEOM) {
                    float dot = 0.0f;
#pragma unroll
                    for (int c = 0; c < CH; ++c) dot = __builtin_fmaf(f[c], grad[k][c], dot);
                    if (rest) dot += rest_dot(b, t.view, s_id[j], fx[k], fy[k], CH);
                    const float la = last_alpha[k];
                    S[k] = __builtin_fmaf(la, last_e[k], S[k]);
                    last_e[k] = dot - S[k];
                    const float grad_alpha = __builtin_fmaf(last_e[k], T[k], bg_t[k] * inv);
                    last_alpha[k] = alpha;
                    // dL/dG = o dL/dalpha; the centre gradient is
                    // -w (a dx + b dy, c dy + b dx) and the conic gradient
                    // -w (dx dx / 2, dx dy, dy dy / 2).
                    const float w = og * grad_alpha;
                    const float ux = __builtin_fmaf(con.x, dx, con.y * dy);
                    const float uy = __builtin_fmaf(con.z, dy, con.y * dx);
                    if (ABS) {
                        const float cx = w * ux, cy = w * uy;
                        vals[0] += cx;
                        vals[1] += cy;
                        vals[6] += __builtin_fabsf(cx);
                        vals[7] += __builtin_fabsf(cy);
                    } else {
                        vals[0] = __builtin_fmaf(w, ux, vals[0]);
                        vals[1] = __builtin_fmaf(w, uy, vals[1]);
                    }
                    const float wx = w * dx, wy = w * dy;
                    vals[2] = __builtin_fmaf(wx, dx, vals[2]);
                    vals[3] = __builtin_fmaf(wx, dy, vals[3]);
                    vals[4] = __builtin_fmaf(wy, dy, vals[4]);
                    vals[5] = __builtin_fmaf(G, grad_alpha, vals[5]);
                }
            }
            if (__ballot(accepted) == 0) continue;
            // Wavefront sums of all gradient entries at once; one atomic
            // instruction, each active lane adding one entry.
            float sums[R];
            wave_sum_rows<NV>(vals, sums);
            // Finish the sums on every lane, ahead of the branch: the last
            // row step then stays one DPP add.
#pragma unroll
            for (int r = 0; r < R; ++r) asm volatile("" : "+v"(sums[r]));
            if (dst_base) {
                const int slot = lane & 15;
                float v = sums[0];
#pragma unroll
                for (int r = 1; r < R; ++r) v = (slot == r) ? sums[r] : v;
                // One 32 x 32 -> 64-bit multiply-add for the address (ids
                // are non-negative, strides below 2^31): 1829 against 1865
                // us for the 3M-Gaussian blend VJP.
                atomicAdd(dst_base + (uint64_t)(uint32_t)s_id[j] * dst_step, v * dst_scale);
            }
          }
        }
    }
}

// Grids of fewer tiles than this (all views) run the narrow-channel blends
// at one pixel per lane: four wavefronts per tile instead of two, so that a
// small frame still spreads over the SIMDs.  Each tile's list is walked
// serially; at two pixels per lane a few thousand tiles make little more than
// one full set of resident wavefronts (6 per SIMD, 6144 on the chip), and the
// longest lists set the time (500K Gaussians at 1280x720, 3600 tiles: a step 0.93 ->
// 0.87 ms at one pixel per lane; 1920x1080, 8160 tiles: 1.31 -> 1.64 ms).
#ifndef GS3D_SMALL_GRID
#define GS3D_SMALL_GRID 4096
#endif
constexpr unsigned kSmallGrid = GS3D_SMALL_GRID;
// Workgroups of a redo launch (gs3d_render_args.redo_pass).
constexpr unsigned kRedoGrid = 512;

template <int CH, int PIX>
int launch_fwd_pix(const gs3d_render_args& a, const gs3d_render_stats_args* st, unsigned long long* counts,
                   unsigned blocks, int c0, hipStream_t s) {
    const dim3 grid(blocks), block(kTilePixels / PIX);
    if (st) {
        const uint32_t kinds = st->sum_mask;
        if (st->requests <= 1) {
            if (kinds & 1u)
                hipLaunchKernelGGL((render_fwd_kernel<CH, PIX, 1, 1, 1>), grid, block, 0, s, a, *st, c0, nullptr);
            else
                hipLaunchKernelGGL((render_fwd_kernel<CH, PIX, 1, 1, 0>), grid, block, 0, s, a, *st, c0, nullptr);
        } else if (st->requests <= 2) {
            switch (kinds & 3u) {
                case 0: hipLaunchKernelGGL((render_fwd_kernel<CH, PIX, 1, 2, 0>), grid, block, 0, s, a, *st, c0, nullptr); break;
                case 1: hipLaunchKernelGGL((render_fwd_kernel<CH, PIX, 1, 2, 1>), grid, block, 0, s, a, *st, c0, nullptr); break;
                case 2: hipLaunchKernelGGL((render_fwd_kernel<CH, PIX, 1, 2, 2>), grid, block, 0, s, a, *st, c0, nullptr); break;
                default: hipLaunchKernelGGL((render_fwd_kernel<CH, PIX, 1, 2, 3>), grid, block, 0, s, a, *st, c0, nullptr); break;
            }
        } else if (st->requests <= 4)
            hipLaunchKernelGGL((render_fwd_kernel<CH, PIX, 1, 4>), grid, block, 0, s, a, *st, c0, nullptr);
        else
            hipLaunchKernelGGL((render_fwd_kernel<CH, PIX, 1, GS3D_MAX_STATISTICS>), grid, block, 0, s, a, *st, c0,
                               nullptr);
        return launch_status("gs3d_render_fwd_stats");
    }
    const gs3d_render_stats_args none = {};
    if (a.redo_pass) {
        // The workgroups walk the listed tiles (usually none).
        hipLaunchKernelGGL((render_fwd_kernel<CH, PIX, 0, 1, -1, 2>), dim3(min(blocks, kRedoGrid)), block, 0, s, a,
                           none, c0, nullptr);
        return launch_status("gs3d_render_fwd");
    }
    if (a.caps || a.stop_out) {
        hipLaunchKernelGGL((render_fwd_kernel<CH, PIX, 0, 1, -1, 1>), grid, block, 0, s, a, none, c0, nullptr);
        return launch_status("gs3d_render_fwd");
    }
    if (counts) {
        hipLaunchKernelGGL((render_fwd_kernel<CH, PIX, 2>), grid, block, 0, s, a, none, c0, counts);
        return launch_status("gs3d_render_pair_counts");
    }
    hipLaunchKernelGGL((render_fwd_kernel<CH, PIX, 0>), grid, block, 0, s, a, none, c0, nullptr);
    return launch_status("gs3d_render_fwd");
}

template <int CH>
int launch_fwd(const gs3d_render_args& a, const gs3d_render_stats_args* st, unsigned long long* counts,
               unsigned blocks, int c0, hipStream_t s) {
    constexpr int PIX = PixFor<CH, false>::value;
    if constexpr (PIX > 1) {
        if (blocks < kSmallGrid) return launch_fwd_pix<CH, 1>(a, st, counts, blocks, c0, s);
    }
    return launch_fwd_pix<CH, PIX>(a, st, counts, blocks, c0, s);
}

// One forward window of `width` channels starting at c0.
inline int launch_fwd_window(const gs3d_render_args& a, const gs3d_render_stats_args* st, unsigned long long* counts,
                             unsigned blocks, int c0, int width, hipStream_t s) {
    if (width <= 4) return launch_fwd<4>(a, st, counts, blocks, c0, s);
    if (width <= 8) return launch_fwd<8>(a, st, counts, blocks, c0, s);
    if (width <= 16) return launch_fwd<16>(a, st, counts, blocks, c0, s);
    if (width <= 36) return launch_fwd<36>(a, st, counts, blocks, c0, s);
    return launch_fwd<kWindow>(a, st, counts, blocks, c0, s);
}

template <int CH, bool GEOM, int PIX>
int launch_bwd_pix(const gs3d_render_bwd_args& b, unsigned blocks, int c0, hipStream_t s) {
    if constexpr (GEOM) {
        if (b.abs_centers) {
            hipLaunchKernelGGL((render_bwd_kernel<CH, true, PIX, true>), dim3(blocks), dim3(kTilePixels / PIX), 0, s, b, c0);
            return launch_status("gs3d_render_bwd");
        }
    }
    hipLaunchKernelGGL((render_bwd_kernel<CH, false, PIX, GEOM>), dim3(blocks), dim3(kTilePixels / PIX), 0, s, b, c0);
    return launch_status("gs3d_render_bwd");
}

template <int CH, bool GEOM>
int launch_bwd(const gs3d_render_bwd_args& b, unsigned blocks, int c0, hipStream_t s) {
    constexpr int PIX = PixFor<CH, true>::value;
    if constexpr (PIX > 1) {
        if (blocks < kSmallGrid) return launch_bwd_pix<CH, GEOM, 1>(b, blocks, c0, s);
    }
    return launch_bwd_pix<CH, GEOM, PIX>(b, blocks, c0, s);
}

inline int check_render_args(const gs3d_render_args& a) {
    if (a.width <= 0 || a.height <= 0 || a.views < 0 || a.n < 0) return GS3D_ERR_ARGUMENT;
    if (a.feat_channels < 0 || a.extra_channels < 0 || (a.extra_channels > 0 && !a.extra)) return GS3D_ERR_ARGUMENT;
    if (a.views > 0 && !a.ranges) return GS3D_ERR_ARGUMENT;
    if (a.views > 0 && a.n > 0 && (!a.centers || !a.conics || (a.feat_channels > 0 && !a.features)))
        return GS3D_ERR_ARGUMENT;
    if ((reinterpret_cast<uintptr_t>(a.centers) & 7) || (reinterpret_cast<uintptr_t>(a.conics) & 15))
        return GS3D_ERR_ARGUMENT;
    const int D = a.feat_channels + a.extra_channels + (a.one_tail ? 1 : 0);
    if (D <= 0) return GS3D_ERR_ARGUMENT;
    return GS3D_OK;
}

inline unsigned render_blocks(const gs3d_render_args& a) {
    const int64_t per_view = (int64_t)((a.width + kTile - 1) / kTile) * ((a.height + kTile - 1) / kTile);
    return (unsigned)(per_view * a.views);
}

}  // namespace gs3d

namespace gs3d {

int render_fwd(const gs3d_render_args* args, const gs3d_render_stats_args* st, unsigned long long* counts,
               void* stream) {
    if (!args) return GS3D_ERR_ARGUMENT;
    const gs3d_render_args& a = *args;
    int status = check_render_args(a);
    if (status != GS3D_OK) return status;
    if (a.zero_count < 0 || (a.zero_count > 0 && (!a.zero_out || (reinterpret_cast<uintptr_t>(a.zero_out) & 15))))
        return GS3D_ERR_ARGUMENT;
    // Capped lists: overflowing tiles must be reported; a redo launch skips
    // tiles, so it cannot clear a buffer, count pairs or total statistics
    // (nor can a capped launch, whose redone tiles would total twice).
    if (a.caps && !a.redo_pass && (!a.redo || !a.redo_list)) return GS3D_ERR_ARGUMENT;
    if (a.redo_pass && (!a.redo_list || a.zero_out)) return GS3D_ERR_ARGUMENT;
    if ((a.caps || a.redo_pass || a.stop_out) && (st || counts)) return GS3D_ERR_ARGUMENT;
    if (a.views == 0) return GS3D_OK;
    if ((a.feat_channels > 0 && !a.image) || (a.extra_channels > 0 && !a.image_extra) ||
        (a.one_tail && !a.image_alpha) || !a.final_t || !a.contributors)
        return GS3D_ERR_ARGUMENT;
    const int D = a.feat_channels + a.extra_channels + (a.one_tail ? 1 : 0);
    const unsigned blocks = render_blocks(a);
    hipStream_t s = as_stream(stream);
    // Windows of up to 64 channels; the statistics ride on window 0.
    for (int c0 = 0; c0 < D; c0 += kWindow) {
        status = launch_fwd_window(a, c0 == 0 ? st : nullptr, c0 == 0 ? counts : nullptr, blocks, c0,
                                   min(kWindow, D - c0), s);
        if (status != GS3D_OK) return status;
    }
    return GS3D_OK;
}

}  // namespace gs3d

extern "C" int gs3d_render_fwd(const gs3d_render_args* args, void* stream) {
    return gs3d::render_fwd(args, nullptr, nullptr, stream);
}

extern "C" int gs3d_render_pair_counts(const gs3d_render_args* args, uint64_t* counts, void* stream) {
    if (!counts || (reinterpret_cast<uintptr_t>(counts) & 7)) return GS3D_ERR_ARGUMENT;
    return gs3d::render_fwd(args, nullptr, reinterpret_cast<unsigned long long*>(counts), stream);
}

extern "C" int gs3d_render_fwd_stats(const gs3d_render_args* args, const gs3d_render_stats_args* stats,
                                     void* stream) {
    if (!args || !stats) return GS3D_ERR_ARGUMENT;
    const gs3d_render_stats_args& st = *stats;
    if (st.requests < 1 || st.requests > GS3D_MAX_STATISTICS) return GS3D_ERR_ARGUMENT;
    const uint32_t used = (1u << st.requests) - 1u;
    if (st.sum_mask & ~used) return GS3D_ERR_ARGUMENT;
    const bool any_sum = st.sum_mask != 0, any_count = st.sum_mask != used;
    if (!st.pixel_values || (any_sum && !st.sums) || (any_count && !st.counts)) return GS3D_ERR_ARGUMENT;
    if (st.pixel_view_stride < 0 || st.counts_view_stride < 0 || st.sums_view_stride < 0) return GS3D_ERR_ARGUMENT;
    if ((reinterpret_cast<uintptr_t>(st.pixel_values) | reinterpret_cast<uintptr_t>(st.counts) |
         reinterpret_cast<uintptr_t>(st.sums)) & 3)
        return GS3D_ERR_ARGUMENT;
    return gs3d::render_fwd(args, stats, nullptr, stream);
}

extern "C" int gs3d_render_bwd(const gs3d_render_bwd_args* args, void* stream) {
    if (!args) return GS3D_ERR_ARGUMENT;
    const gs3d_render_bwd_args& b = *args;
    const gs3d_render_args& a = b.fwd;
    int status = gs3d::check_render_args(a);
    if (status != GS3D_OK) return status;
    if (a.views == 0) return GS3D_OK;
    if (!a.final_t || !a.contributors || !b.grad_centers || !b.grad_conics) return GS3D_ERR_ARGUMENT;
    if (b.grad_centers_stride < 2 || b.grad_conics_stride < 4 || (b.abs_centers && b.abs_stride < 2))
        return GS3D_ERR_ARGUMENT;
    // Gradient row strides feed 32-bit multipliers in the kernel.
    for (int64_t stride : {b.grad_centers_stride, b.grad_conics_stride, b.abs_stride, b.grad_feat_stride,
                           b.grad_extra_stride})
        if (stride < 0 || stride > INT32_MAX) return GS3D_ERR_ARGUMENT;
    if ((b.upstream && b.upstream_stride < a.feat_channels) ||
        (b.upstream_extra && b.upstream_extra_stride < a.extra_channels) ||
        (b.upstream_alpha && b.upstream_alpha_stride < 1))
        return GS3D_ERR_ARGUMENT;
    using namespace gs3d;
    const int D = a.feat_channels + a.extra_channels + (a.one_tail ? 1 : 0);
    const int Dg = D - (a.one_tail ? 1 : 0);
    const unsigned blocks = render_blocks(a);
    hipStream_t s = as_stream(stream);
    // Geometry launch over the first window (channels beyond it enter its
    // alpha gradient from global memory), then the feature gradients of the
    // further windows that hold channels with a destination.
    if (D <= 4) status = launch_bwd<4, true>(b, blocks, 0, s);
    else if (D <= 8) status = launch_bwd<8, true>(b, blocks, 0, s);
    else if (D <= 16) status = launch_bwd<16, true>(b, blocks, 0, s);
    else if (D <= 36) status = launch_bwd<36, true>(b, blocks, 0, s);
    else status = launch_bwd<kGeomWindow, true>(b, blocks, 0, s);
    if (status != GS3D_OK || (!b.grad_features && !b.grad_extra)) return status;
    for (int c0 = kGeomWindow; c0 < Dg; c0 += kWindow) {
        const int width = min(kWindow, D - c0);
        if (width <= 4) status = launch_bwd<4, false>(b, blocks, c0, s);
        else if (width <= 8) status = launch_bwd<8, false>(b, blocks, c0, s);
        else if (width <= 16) status = launch_bwd<16, false>(b, blocks, c0, s);
        else if (width <= 36) status = launch_bwd<36, false>(b, blocks, c0, s);
        else status = launch_bwd<kWindow, false>(b, blocks, c0, s);
        if (status != GS3D_OK) return status;
    }
    return GS3D_OK;
}
