// Tile binning: inclusive scan of tile counts, (tile << 32 | depth bits) key
// emission, stable LSD radix sort of (key, id) pairs and per-tile ranges.
//
// primitives/tiling.py:28-100 (float_bits, sort_key, identify_ranges,
// scan_counts, sort_tile_pairs) and splatting/binning.py:16-37, :71-117
// (duplicate, bin_and_sort).  All of it is integer work over HBM-resident
// arrays: coalesced loads, LDS-local reordering before every scatter, no
// matrix cores.
#include <climits>

#include <type_traits>
#include <utility>
#include <mutex>

#include "common.hpp"
#include "footprint.hpp"

namespace gs3d {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;

// ---------------------------------------------------------------------------
// Block-level helpers
// ---------------------------------------------------------------------------
// Inclusive scan across a wavefront (shuffle-up).
template <class T>
GS3D_DEV T wave_inclusive_scan(T v) {
    const int lane = lane_id();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const T u = __shfl_up(v, d, 64);
        if (lane >= d) v += u;
    }
    return v;
}

// Exclusive scan across the block (B threads); returns the block total too.
template <int B, class T>
GS3D_DEV T block_exclusive_scan(T v, T* s_wave, T& total) {
    constexpr int W = B / 64;
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    const T inc = wave_inclusive_scan(v);
    if (lane == 63) s_wave[wave] = inc;
    __syncthreads();
    T before = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < W; ++w) {
        const T x = s_wave[w];
        before += (w < wave) ? x : T(0);
        sum += x;
    }
    __syncthreads();
    total = sum;
    return before + inc - v;
}

// A sum of int64 values that a scan's first launch adds up beside its own
// work (in one more workgroup, or in its single workgroup before the scan),
// so that a sum too small to fill the GPU costs no launch of its own.
struct SideSum {
    const int64_t* values = nullptr;
    int64_t count = 0;
    int64_t* out = nullptr;
};

// *side.out = sum of side.values[0, count), by the whole block of B threads;
// eight loads per thread in flight at a time.
template <int B>
GS3D_DEV void side_sum(const SideSum& side, int64_t* s_wave) {
    constexpr int U = 8;
    int64_t v = 0;
    for (int64_t i0 = threadIdx.x; i0 < side.count; i0 += (int64_t)B * U) {
        int64_t x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + (int64_t)u * B;
            x[u] = i < side.count ? side.values[i] : 0;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) v += x[u];
    }
    int64_t total;
    block_exclusive_scan<B>(v, s_wave, total);
    if (threadIdx.x == 0) *side.out = total;
}

// ---------------------------------------------------------------------------
// Scan (reduce-then-scan over 4096-element tiles).
// ---------------------------------------------------------------------------
// One wavefront per 4096-element tile: all 64 loads of a lane in flight at
// once, then a butterfly sum (no LDS, no block barrier).
constexpr int kReduceWaves = 4;
template <class In>
__global__ __launch_bounds__(64 * kReduceWaves) void scan_reduce_kernel(const In* __restrict__ in, int64_t n,
                                                                        int64_t tiles,
                                                                        int64_t* __restrict__ partials,
                                                                        SideSum side) {
    if (side.values && blockIdx.x == gridDim.x - 1) {  // the extra workgroup
        __shared__ int64_t s_wave[kReduceWaves];
        side_sum<64 * kReduceWaves>(side, s_wave);
        return;
    }
    const int lane = lane_id();
    const int64_t tile = (int64_t)blockIdx.x * kReduceWaves + (threadIdx.x >> 6);
    if (tile >= tiles) return;
    const int64_t base = tile * kScanTile;
    constexpr int kPerLane = kScanTile / 64;
    // Clamped addresses and a select keep every load unconditional (a
    // guarded load is a branch that waits for its data).
    In v[kPerLane];
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) {
        const int64_t idx = base + k * 64 + lane;
        v[k] = in[min(idx, n - 1)];
    }
#pragma unroll
    for (int k = 0; k < kPerLane; ++k)
        if (base + k * 64 + lane >= n) v[k] = In(0);
    int64_t sum = 0;
#pragma unroll
    for (int k = 0; k < kPerLane; ++k) sum += (int64_t)v[k];
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) sum += __shfl_xor(sum, d, 64);
    if (lane == 0) partials[tile] = sum;
}

// Per-tile scan with the tile's prefix.  Loads and stores are striped
// across the block (coalesced) and transposed through LDS so that each thread
// scans 16 consecutive elements; the LDS index e + e/16 keeps both the
// striped and the per-thread accesses free of bank conflicts.
GS3D_DEV int scan_lds_index(int e) { return e + (e >> 4); }

// The tile's prefix is the sum of the earlier tiles' totals, which every
// block adds up itself (a few thousand L2-resident values at most), so no
// separate launch scans the totals.  The last block writes the grand total.
template <class In, bool INCLUSIVE>
__global__ __launch_bounds__(kScanThreads) void scan_down_kernel(const In* __restrict__ in, int64_t n,
                                                                 const int64_t* __restrict__ partials,
                                                                 int32_t* __restrict__ out,
                                                                 int64_t* __restrict__ total_out) {
    __shared__ int64_t s_wave[kScanThreads / 64];
    __shared__ int32_t s_tile[kScanTile + kScanTile / 16];
    const int64_t base = (int64_t)blockIdx.x * kScanTile;
    // The tile's loads are issued first: they overlap the prefix's.
    int32_t raw[kScanItems];
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) raw[k] = (int32_t)in[min(base + k * kScanThreads + threadIdx.x, n - 1)];
#pragma unroll
    for (int k = 0; k < kScanItems; ++k)
        if (base + k * kScanThreads + threadIdx.x >= n) raw[k] = 0;
    int64_t before = 0;
    for (int64_t j0 = threadIdx.x; j0 < (int64_t)blockIdx.x; j0 += 4 * kScanThreads) {
        int64_t p[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) p[u] = partials[min(j0 + u * kScanThreads, (int64_t)blockIdx.x - 1)];
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (j0 + u * kScanThreads >= (int64_t)blockIdx.x) p[u] = 0;
        before += (p[0] + p[1]) + (p[2] + p[3]);
    }
    int64_t prefix;
    block_exclusive_scan<kScanThreads>(before, s_wave, prefix);
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) s_tile[scan_lds_index(k * kScanThreads + threadIdx.x)] = raw[k];
    __syncthreads();
    int32_t vals[kScanItems];
    int64_t sum = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        vals[k] = s_tile[scan_lds_index(threadIdx.x * kScanItems + k)];
        sum += vals[k];
    }
    int64_t total;
    int64_t run = block_exclusive_scan<kScanThreads>(sum, s_wave, total) + prefix;
    if (total_out && blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) *total_out = prefix + total;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        if (INCLUSIVE) run += vals[k];
        s_tile[scan_lds_index(threadIdx.x * kScanItems + k)] = (int32_t)run;
        if (!INCLUSIVE) run += vals[k];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        const int e = k * kScanThreads + threadIdx.x;
        const int64_t idx = base + e;
        if (idx < n) out[idx] = s_tile[scan_lds_index(e)];
    }
}

// Small scans in one workgroup: up to kSingleScanMax entries, tiles of
// kSingleTile with a running carry.  One launch instead of two (three with
// the radix sort's transpose, which it can write directly): at these sizes
// every launch costs more than the work it does.  With rows > 0, `in` is a
// [cols][rows] table (entry e = c * rows + r) and out[r * cols + c] receives
// entry e's scan: the transposed layout the sort scatter reads.
constexpr int kSingleThreads = 512;
constexpr int kSingleItems = 16;
constexpr int kSingleTile = kSingleThreads * kSingleItems;
// Measured: at 1-2 tiles one launch of this kernel (4-5 us) replaces two or
// three (3-5 us each); at 8 tiles it is slower than the grid-wide scan.
constexpr int64_t kSingleScanMax = 2 * kSingleTile;

template <class In, bool INCLUSIVE>
__global__ __launch_bounds__(kSingleThreads) void scan_single_kernel(const In* __restrict__ in, int64_t n,
                                                                     int32_t* __restrict__ out,
                                                                     int64_t* __restrict__ total_out, int32_t rows,
                                                                     int32_t cols, SideSum side) {
    __shared__ int64_t s_wave[kSingleThreads / 64];
    __shared__ int32_t s_tile[kSingleTile + kSingleTile / 16];
    if (side.values) side_sum<kSingleThreads>(side, s_wave);
    const int count = (int)n;  // n <= kSingleScanMax
    int64_t carry = 0;
    for (int base = 0; base < count; base += kSingleTile) {
        int32_t raw[kSingleItems];
#pragma unroll
        for (int k = 0; k < kSingleItems; ++k) raw[k] = (int32_t)in[min(base + k * kSingleThreads + (int)threadIdx.x, count - 1)];
#pragma unroll
        for (int k = 0; k < kSingleItems; ++k) {
            const int e = k * kSingleThreads + (int)threadIdx.x;
            s_tile[scan_lds_index(e)] = base + e < count ? raw[k] : 0;
        }
        __syncthreads();
        int32_t vals[kSingleItems];
        int64_t sum = 0;
#pragma unroll
        for (int k = 0; k < kSingleItems; ++k) {
            vals[k] = s_tile[scan_lds_index((int)threadIdx.x * kSingleItems + k)];
            sum += vals[k];
        }
        int64_t tile_total;
        int64_t run = block_exclusive_scan<kSingleThreads>(sum, s_wave, tile_total) + carry;
#pragma unroll
        for (int k = 0; k < kSingleItems; ++k) {
            if (INCLUSIVE) run += vals[k];
            s_tile[scan_lds_index((int)threadIdx.x * kSingleItems + k)] = (int32_t)run;
            if (!INCLUSIVE) run += vals[k];
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kSingleItems; ++k) {
            const int e = k * kSingleThreads + (int)threadIdx.x;
            const int idx = base + e;
            if (idx < count) {
                const int32_t v = s_tile[scan_lds_index(e)];
                if (rows > 0) {
                    const int c = idx / rows, r = idx - c * rows;
                    out[(int64_t)r * cols + c] = v;
                } else {
                    out[idx] = v;
                }
            }
        }
        carry += tile_total;
        __syncthreads();  // the next tile reuses s_tile
    }
    if (total_out && threadIdx.x == 0) *total_out = carry;
}

inline size_t scan_partials_bytes(int64_t n) {
    const int64_t tiles = (n + kScanTile - 1) / kScanTile;
    return (size_t)((tiles + 1) * sizeof(int64_t) + 255) & ~(size_t)255;
}

// Scratch layout: [tile totals (tiles int64)].  side (optional): a sum the
// first launch also computes.
template <class In, bool INCLUSIVE>
int run_scan(const In* in, int64_t n, int32_t* out, int64_t* total, void* scratch, hipStream_t stream,
             SideSum side = SideSum{}) {
    const int64_t tiles = (n + kScanTile - 1) / kScanTile;
    if (tiles == 0 && !side.values) return GS3D_OK;  // callers handle empty inputs (total untouched)
    if (n <= kSingleScanMax) {
        hipLaunchKernelGGL((scan_single_kernel<In, INCLUSIVE>), dim3(1), dim3(kSingleThreads), 0, stream, in, n, out,
                           n > 0 ? total : nullptr, 0, 0, side);
        return launch_status("scan");
    }
    int64_t* partials = reinterpret_cast<int64_t*>(scratch);
    const unsigned reduce_blocks = (unsigned)((tiles + kReduceWaves - 1) / kReduceWaves) + (side.values ? 1u : 0u);
    hipLaunchKernelGGL((scan_reduce_kernel<In>), dim3(reduce_blocks), dim3(64 * kReduceWaves), 0, stream, in, n,
                       tiles, partials, side);
    hipLaunchKernelGGL((scan_down_kernel<In, INCLUSIVE>), dim3((unsigned)tiles), dim3(kScanThreads), 0, stream, in, n,
                       partials, out, total);
    return launch_status("scan");
}

// ---------------------------------------------------------------------------
// Key emission (splatting/binning.py:16-37).  Rows touching at most
// kSmallRect tiles emit their pairs serially; larger rows are queued and a
// whole block writes each one (coalesced, balanced across the grid).
// ---------------------------------------------------------------------------
constexpr int kSmallRect = 32;
constexpr int kEmitThreads = 256;

GS3D_DEV uint64_t make_key(uint32_t tile, float depth) {
    return ((uint64_t)tile << 32) | (uint64_t)__float_as_uint(depth);
}

__global__ void fill_u32_kernel(uint32_t* p, int64_t count, uint32_t value) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = value;
}

// Fill kernel launch (no memset nodes, so the sequence stays capturable).
inline void fill_u32(uint32_t* p, int64_t count, uint32_t value, hipStream_t s) {
    if (count <= 0) return;
    const int64_t blocks = (count + 255) / 256;
    hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, s, p, count,
                       value);
}

// Tile rectangle of row r in the rectangle modes (radius square or SnugBox).
GS3D_DEV int4 emit_rect(const gs3d_emit_args& a, int64_t r, int radius, int gx, int gy) {
    const float2 c = reinterpret_cast<const float2*>(a.centers)[r];
    const float4 k = a.tile_mode == GS3D_TILE_RADIUS ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
                                                     : reinterpret_cast<const float4*>(a.conics)[r];
    int4 rect = mode_rect(c, k, radius, gx, gy, a.tile_mode);
    rect.z = max(rect.z, rect.x);
    rect.w = max(rect.w, rect.y);
    return rect;
}

__global__ __launch_bounds__(kEmitThreads) void emit_small_kernel(gs3d_emit_args a, uint32_t* __restrict__ queue_count,
                                                                  int32_t* __restrict__ queue) {
    const int64_t rows = (int64_t)a.n * a.views;
    const int64_t r = (int64_t)blockIdx.x * kEmitThreads + threadIdx.x;
    if (r >= rows) return;
    const int radius = a.radii[r];
    if (radius <= 0) return;
    const int gx = (a.width + 15) / 16, gy = (a.height + 15) / 16;
    const int4 rect = emit_rect(a, r, radius, gx, gy);
    const int w = rect.z - rect.x;
    const int64_t off0 = r > 0 ? a.offsets[r - 1] : 0;
    // The slot reserved by the scan bounds the emission (equal by construction).
    const int count = (int)min((int64_t)(w * (rect.w - rect.y)), (int64_t)a.offsets[r] - off0);
    if (count <= 0) return;
    if (count > kSmallRect) {
        const uint32_t slot = atomicAdd(queue_count, 1u);
        queue[slot] = (int32_t)r;
        return;
    }
    const int64_t view = r / a.n;
    const int32_t id = (int32_t)(r - view * a.n);
    const uint32_t tile0 = (uint32_t)(view * gx * gy);
    const uint32_t bits = __float_as_uint(a.depths[r]);
    int k = 0;
    for (int y = rect.y; y < rect.w && k < count; ++y)
        for (int x = rect.x; x < rect.z && k < count; ++x, ++k) {
            a.keys[off0 + k] = ((uint64_t)(tile0 + (uint32_t)(y * gx + x)) << 32) | (uint64_t)bits;
            a.values[off0 + k] = id;
        }
}

__global__ __launch_bounds__(kEmitThreads) void emit_large_kernel(gs3d_emit_args a,
                                                                  const uint32_t* __restrict__ queue_count,
                                                                  const int32_t* __restrict__ queue) {
    const uint32_t total = *queue_count;
    const int gx = (a.width + 15) / 16, gy = (a.height + 15) / 16;
    for (uint32_t q = blockIdx.x; q < total; q += gridDim.x) {
        const int64_t r = queue[q];
        const int4 rect = emit_rect(a, r, a.radii[r], gx, gy);
        const int w = rect.z - rect.x;
        const int64_t off = r > 0 ? a.offsets[r - 1] : 0;
        const int count = (int)min((int64_t)(w * (rect.w - rect.y)), (int64_t)a.offsets[r] - off);
        const int64_t view = r / a.n;
        const int32_t id = (int32_t)(r - view * a.n);
        const uint32_t tile0 = (uint32_t)(view * gx * gy);
        const uint32_t bits = __float_as_uint(a.depths[r]);
        for (int k = threadIdx.x; k < count; k += kEmitThreads) {
            const int dy = k / w, dx = k - dy * w;
            const uint32_t tile = tile0 + (uint32_t)((rect.y + dy) * gx + rect.x + dx);
            a.keys[off + k] = ((uint64_t)tile << 32) | (uint64_t)bits;
            a.values[off + k] = id;
        }
    }
}

// AccuTile emission (splatting/binning.py:40-68 with intersections.py:160-218):
// one thread per row writes its strips' tiles in traversal order.
__global__ __launch_bounds__(kEmitThreads) void emit_accutile_kernel(gs3d_emit_args a) {
    const int64_t rows = (int64_t)a.n * a.views;
    const int64_t r = (int64_t)blockIdx.x * kEmitThreads + threadIdx.x;
    if (r >= rows) return;
    const int radius = a.radii[r];
    if (radius <= 0) return;
    const int64_t off = r > 0 ? a.offsets[r - 1] : 0;
    const int64_t reserved = (int64_t)a.offsets[r] - off;
    if (reserved <= 0) return;
    const int gx = (a.width + 15) / 16, gy = (a.height + 15) / 16;
    const Ellipse e = footprint(reinterpret_cast<const float2*>(a.centers)[r], reinterpret_cast<const float4*>(a.conics)[r],
                                radius, gx, gy);
    const int64_t view = r / a.n;
    const int32_t id = (int32_t)(r - view * a.n);
    const uint32_t tile0 = (uint32_t)(view * gx * gy);
    const uint32_t bits = __float_as_uint(a.depths[r]);
    int64_t k = 0;
    bool is_y = true;
    accutile_strips(e, is_y, [&](int row, int lo, int hi) {
        for (int col = lo; col < hi; ++col, ++k) {
            if (k >= reserved) continue;
            const uint32_t tile = tile0 + (uint32_t)(is_y ? row * gx + col : col * gx + row);
            a.keys[off + k] = ((uint64_t)tile << 32) | (uint64_t)bits;
            a.values[off + k] = id;
        }
    });
}

// ---------------------------------------------------------------------------
// LSD radix sort of (key, int32 value) pairs, 8-bit digits, for 32- and
// 64-bit keys.  Per pass: per-tile digit histograms (digit-major
// [256][tiles]), one exclusive scan over them (the scatter base of every
// (digit, tile)), then a stable rank-and-scatter: each wavefront ranks its
// 512 keys with ballot-based digit matching, the block orders its 2048 keys
// by digit in LDS and writes them out in digit runs (coalesced).
// ---------------------------------------------------------------------------
constexpr int kSortThreads = 256;
#ifndef GS3D_SORT_ITEMS
#define GS3D_SORT_ITEMS 8
#endif
constexpr int kSortItems = GS3D_SORT_ITEMS;  // keys per thread of a sort tile
constexpr int kSortTile = kSortThreads * kSortItems;  // 2048 keys
constexpr int kRadix = 256;
#ifndef GS3D_SORT_XCD
#define GS3D_SORT_XCD 1
#endif
#ifndef GS3D_HIST_TILES8
#define GS3D_HIST_TILES8 4
#endif

// Workgroups are dispatched to the 8 XCDs in turn; giving every XCD one
// contiguous range of logical blocks keeps consecutive chunks of a group --
// and so the consecutive segments of its tiles' lists -- in one L2.
GS3D_DEV int64_t xcd_contiguous(int64_t b, int64_t nblocks) {
    constexpr int64_t kXcds = 8;
    const int64_t per = nblocks / kXcds, rem = nblocks % kXcds;
    const int64_t xcd = b % kXcds, k = b / kXcds;
    return xcd * per + min(xcd, rem) + k;
}

template <class K>
GS3D_DEV uint32_t digit_of(K key, int shift, uint32_t mask) { return (uint32_t)(key >> shift) & mask; }

// Outputs of the depth order's last pass (TAIL != 0): the group count of
// every record at its sorted position and each block's tile-pair sum, taken
// from the packed record (TAIL 1: tile rectangle, TAIL 2: AccuTile
// tiles << 12 | groups).  The counts are 16-bit: a packed rectangle spans at
// most 32 x 32 groups and an AccuTile record holds fewer than 4096.
struct OrderTail {
    uint16_t* group_counts;
    int64_t* block_pairs;
};
template <int TAIL>
GS3D_DEV void record_extent(uint64_t record, int32_t& groups, int64_t& area);

// Rows that the depth order leaves out: they touch no tile group, and
// row_records_kernel gives them the key kDroppedKey (a NaN pattern, never the
// depth bits of a projected row).  The first pass (DROP) neither counts nor
// places such keys; `live` (device memory, from that pass's digit scan) is
// then the number of keys the later passes sort, and the last pass (`fill`)
// writes `filler` into every position of [live, count).
constexpr uint32_t kDroppedKey = 0xFFFFFFFFu;
struct Culled {
    const int64_t* live;  // null: every key of [0, count) is sorted
    bool fill;
    uint64_t filler;
    // Optional: digits are taken from key - *key_base (every key sorted is at
    // least *key_base, so the order is unchanged and the difference may need
    // fewer bits than the key).
    const uint32_t* key_base = nullptr;
};

// VALS = false sorts keys alone: no value loads, stores or LDS staging, which
// leaves room for one more block per CU.  R: the digits the LDS counters hold
// (every key's digit is below it; fewer than 1 << RB when the keys are known
// to stay below R, which leaves more LDS for resident blocks).
template <class K, class V, bool VALS, int RB = 8, int TAIL = 0, bool DROP = false, int R = 1 << RB>
__global__ __launch_bounds__(kSortThreads) void sort_scatter_kernel(
    const K* __restrict__ keys_in, const V* __restrict__ vals_in, K* __restrict__ keys_out,
    V* __restrict__ vals_out, int64_t count, int shift, uint32_t mask, int bits,
    const int32_t* __restrict__ offsets, int64_t tiles, int digits, OrderTail tail, Culled cull) {
    static_assert(TAIL == 0 || (VALS && sizeof(V) == 8), "the order tail reads 64-bit records");
    static_assert(R % kSortThreads == 0 && R <= (1 << RB), "whole digits per thread");
    __shared__ K s_keys[kSortTile];
    __shared__ V s_vals[VALS ? kSortTile : 1];
    __shared__ uint32_t s_wcnt[kSortThreads / 64][R];
    __shared__ int32_t s_gbase[R];
    __shared__ uint32_t s_scan_wave[kSortThreads / 64];
    const int wave = threadIdx.x >> 6, lane = lane_id();
    for (int e = threadIdx.x; e < (kSortThreads / 64) * R; e += kSortThreads) (&s_wcnt[0][0])[e] = 0;
    // Consecutive tiles on one XCD: their runs of the same digit are adjacent
    // in the output, and partial lines merge in that XCD's L2.
    const int64_t tile = GS3D_SORT_XCD ? xcd_contiguous(blockIdx.x, gridDim.x) : (int64_t)blockIdx.x;
    const int64_t tile_base = tile * kSortTile;
    const int64_t live = cull.live ? min(count, *cull.live) : count;
    const K key_base = cull.key_base ? (K)*cull.key_base : K(0);
    auto digit = [&](K k) { return digit_of((K)(k - key_base), shift, mask); };
    K key[kSortItems];
    V val[kSortItems];
    uint32_t rank[kSortItems];
    bool in[kSortItems];  // the key takes part in this pass
    // This tile's global digit offsets (thread t owns the M consecutive
    // digits from M t), loaded now so that they arrive during the ranking.
    constexpr int M = R / kSortThreads;
    int32_t digit_offset[M];
#pragma unroll
    for (int i = 0; i < M; ++i) {
        const int d = threadIdx.x * M + i;
        digit_offset[i] = offsets[tile * digits + min(d, digits - 1)];
    }
    const int64_t base = tile_base + wave * (kSortTile / 4) + lane;
#pragma unroll
    for (int k = 0; k < kSortItems; ++k) {
        const int64_t idx = base + k * 64;
        if (idx < live) {
            key[k] = keys_in[idx];
            val[k] = VALS ? vals_in[idx] : V(0);
        } else {
            key[k] = K(0);
            val[k] = V(0);
        }
        in[k] = idx < live && !(DROP && key[k] == (K)kDroppedKey);
    }
    __syncthreads();
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
    for (int k = 0; k < kSortItems; ++k) {
        rank[k] = 0;
        if (in[k]) {
            const uint32_t d = digit(key[k]);
            uint64_t peers = __ballot(1);
            for (int b = 0; b < bits; ++b) {
                const bool set = (d >> b) & 1u;
                const uint64_t m = __ballot(set);
                peers &= set ? m : ~m;
            }
            const uint32_t before = (uint32_t)__popcll(peers & lt_mask);
            const uint32_t start = s_wcnt[wave][d];
            rank[k] = start + before;
            const int last = 63 - __clzll(peers);
            if (lane == last) s_wcnt[wave][d] = start + (uint32_t)__popcll(peers);
        }
    }
    __syncthreads();
    uint32_t block_total;  // keys of this tile taking part in the pass
    {
        // Start of digit d in this tile's digit-sorted order, then each
        // wavefront's offset within the digit.
        uint32_t c[M][kSortThreads / 64];
        uint32_t tot = 0;
#pragma unroll
        for (int i = 0; i < M; ++i) {
#pragma unroll
            for (int w = 0; w < kSortThreads / 64; ++w) {
                c[i][w] = s_wcnt[w][threadIdx.x * M + i];
                tot += c[i][w];
            }
        }
        uint32_t run = block_exclusive_scan<kSortThreads>(tot, s_scan_wave, block_total);
#pragma unroll
        for (int i = 0; i < M; ++i) {
            const int d = threadIdx.x * M + i;
            // Digits at or beyond `digits` (the offsets' row length) hold no key.
            s_gbase[d] = d < digits ? digit_offset[i] - (int32_t)run : 0;
#pragma unroll
            for (int w = 0; w < kSortThreads / 64; ++w) {
                s_wcnt[w][d] = run;
                run += c[i][w];
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kSortItems; ++k) {
        if (in[k]) {
            const uint32_t d = digit(key[k]);
            const uint32_t pos = s_wcnt[wave][d] + rank[k];
            s_keys[pos] = key[k];
            if (VALS) s_vals[pos] = val[k];
        }
    }
    __syncthreads();
    int64_t area_sum = 0;
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int p = j * kSortThreads + threadIdx.x;
        if (p < (int)block_total) {
            const K kk = s_keys[p];
            const int64_t dst = (int64_t)s_gbase[digit(kk)] + p;
            keys_out[dst] = kk;  // plain stores: digit runs start mid-line and the L2 merges them
            if (VALS) vals_out[dst] = s_vals[p];
            if constexpr (TAIL != 0) {
                int32_t groups;
                int64_t area;
                record_extent<TAIL>((uint64_t)s_vals[p], groups, area);
                tail.group_counts[dst] = (uint16_t)groups;
                area_sum += area;
            }
        }
    }
    if constexpr (VALS) {
        if (cull.fill && cull.live) {
            // This tile's share of the positions after the sorted keys.
#pragma unroll
            for (int j = 0; j < kSortItems; ++j) {
                const int64_t q = tile_base + j * kSortThreads + threadIdx.x;
                if (q >= live && q < count) {
                    vals_out[q] = (V)cull.filler;
                    if constexpr (TAIL != 0) tail.group_counts[q] = 0;
                }
            }
        }
    }
    if constexpr (TAIL != 0) {
        __shared__ int64_t s_area[kSortThreads / 64];
        int64_t total;
        block_exclusive_scan<kSortThreads>(area_sum, s_area, total);
        if (threadIdx.x == 0) tail.block_pairs[blockIdx.x] = total;
    }
}

// Digit counts of the radix sort: a [digit][tile] table (the order in which a
// stable LSD pass places the keys, so its flat exclusive scan gives every
// tile's offset for every digit), written by histogram blocks of several
// consecutive tiles (runs of words instead of one scattered word per digit).
// The scan is written transposed, [tile][digit], so that each scatter block
// reads its offsets as one contiguous row.
struct SortScratch {
    uint16_t* counts;     // [R][tiles], each at most kSortTile (its region keeps room for 32-bit words)
    int32_t* offsets;     // [tiles][R], the exclusive scan of counts in digit-major order
    int32_t* scan;        // the digit scan's segment prefixes [R][segments] and row totals [R]
};

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

constexpr int kSegTiles = 128;  // tiles per segment of the digit scan

inline size_t sort_scratch_bytes(int64_t count, SortScratch* out, void* base, int radix_bits = 8) {
    const int64_t tiles = (count + kSortTile - 1) / kSortTile;
    const int64_t segs = (tiles + kSegTiles - 1) / kSegTiles;
    const size_t a = align256((size_t)(tiles << radix_bits) * 4);
    const size_t b = align256((size_t)((segs + 1) << radix_bits) * 4);
    if (out) {
        char* p = reinterpret_cast<char*>(base);
        out->counts = reinterpret_cast<uint16_t*>(p);
        out->offsets = reinterpret_cast<int32_t*>(p + a);
        out->scan = reinterpret_cast<int32_t*>(p + 2 * a);
    }
    return 2 * a + b;
}

// Digit scan of a sort pass in two launches.  The exclusive scan of the
// digit-major count table counts[d][t] is written transposed, as the
// offsets[t][d] the scatter reads (each tile's base for every digit):
//   digit_rows_kernel: one workgroup per digit row adds up the row in
//     segments of kSegTiles tiles and writes each segment's exclusive prefix
//     within the row (seg_prefix[d][segment]) and the row's total;
//   digit_offsets_kernel: one workgroup per kSegDigits digits x kSegTiles
//     tiles scans its block in LDS from the totals of the rows above and the
//     segment prefixes, and writes it transposed (128-byte rows).
// No workgroup waits for another and the scanned table is never stored
// digit-major.
constexpr int kSegDigits = 32;
constexpr int kRowThreads = 256;

// Each wavefront owns ITEMS / 2 consecutive segments of a chunk of
// kRowThreads * ITEMS tiles (every load a run of 64 words); a lane adds its
// two words of a segment before the wave sum.  Small workgroups keep every
// row of the table resident at once (up to 1024 rows), and ITEMS (chosen
// from the row length) puts a whole row in one chunk up to 12288 tiles.
template <int ITEMS>
__global__ __launch_bounds__(kRowThreads) void digit_rows_kernel(const uint16_t* __restrict__ counts, int tiles,
                                                                 int segs, int32_t* __restrict__ seg_prefix,
                                                                 int32_t* __restrict__ row_totals) {
    static_assert(ITEMS % 2 == 0, "two words of a segment per lane");
    constexpr int kChunkTiles = kRowThreads * ITEMS;
    constexpr int kChunkSegs = kChunkTiles / kSegTiles;
    constexpr int kWaveSegs = ITEMS / 2;
    __shared__ uint32_t s_seg[kChunkSegs];
    const int d = blockIdx.x;
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    const uint16_t* row = counts + (int64_t)d * tiles;
    int64_t carry = 0;  // wave 0: the row's sum before this chunk
    for (int c0 = 0; c0 < tiles; c0 += kChunkTiles) {
        const int w0 = c0 + wave * (ITEMS * 64) + lane;
        uint32_t v[ITEMS];
#pragma unroll
        for (int m = 0; m < ITEMS; ++m) v[m] = row[min(w0 + m * 64, tiles - 1)];
#pragma unroll
        for (int m = 0; m < ITEMS; ++m)
            if (w0 + m * 64 >= tiles) v[m] = 0;
#pragma unroll
        for (int s = 0; s < kWaveSegs; ++s) {
            const uint32_t sum = wave_sum_u32_to_lane63(v[2 * s] + v[2 * s + 1]);
            if (lane == 63) s_seg[wave * kWaveSegs + s] = sum;
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int g = 0; g < (kChunkSegs + 63) / 64; ++g) {
                const int j = g * 64 + lane;
                const uint32_t s = j < kChunkSegs ? s_seg[j] : 0u;
                const uint32_t inc = wave_inclusive_scan(s);
                const int seg = c0 / kSegTiles + j;
                if (j < kChunkSegs && seg < segs)
                    seg_prefix[(int64_t)d * segs + seg] = (int32_t)(carry + (int64_t)(inc - s));
                carry += (int64_t)__shfl(inc, 63, 64);
            }
        }
        __syncthreads();  // the next chunk reuses s_seg
    }
    if (threadIdx.x == 0) row_totals[d] = (int32_t)carry;
}

template <int ITEMS>
void launch_digit_rows(int per_thread, int digits, const uint16_t* counts, int tiles, int segs, int32_t* seg_prefix,
                       int32_t* row_totals, hipStream_t s) {
    if constexpr (ITEMS < 48) {
        if (per_thread > ITEMS)
            return launch_digit_rows<ITEMS + 8>(per_thread, digits, counts, tiles, segs, seg_prefix, row_totals, s);
    }
    hipLaunchKernelGGL(digit_rows_kernel<ITEMS>, dim3((unsigned)digits), dim3(kRowThreads), 0, s, counts, tiles, segs,
                       seg_prefix, row_totals);
}

// grid (segments, digits / kSegDigits); total_out (optional) receives the
// sum of the table.
__global__ __launch_bounds__(256) void digit_offsets_kernel(const uint16_t* __restrict__ counts, int64_t tiles,
                                                            int digits, const int32_t* __restrict__ seg_prefix,
                                                            const int32_t* __restrict__ row_totals,
                                                            int32_t* __restrict__ offsets,
                                                            int64_t* __restrict__ total_out) {
    static_assert(kSegTiles == 128 && kSegDigits == 32, "the thread mapping below");
    __shared__ int32_t s_block[kSegDigits][kSegTiles + 1];
    __shared__ int32_t s_row[kSegDigits];
    __shared__ int64_t s_wave[4];
    const int64_t segs = gridDim.x, seg = blockIdx.x;
    const int64_t t0 = seg * kSegTiles;
    const int d0 = blockIdx.y * kSegDigits;
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    // Every load is issued before the first wait: the block's rows (lanes
    // 0-31 of wave 0: total and segment prefix of row d0 + lane), its counts
    // (entry k * 256 + thread is row 2k + thread / 128 of the block, column
    // thread % 128) and the totals of the rows above it.
    int64_t rt = 0;
    int32_t sp = 0;
    if (wave == 0 && lane < kSegDigits) {
        rt = row_totals[d0 + lane];
        sp = seg_prefix[(int64_t)(d0 + lane) * segs + seg];
    }
    const int col = threadIdx.x & (kSegTiles - 1), half = threadIdx.x >> 7;
    const int64_t t = t0 + col;
    uint32_t raw[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) raw[k] = counts[(int64_t)(d0 + 2 * k + half) * tiles + min(t, tiles - 1)];
    int64_t above = 0;
    for (int j = threadIdx.x; j < d0; j += 256) above += row_totals[j];
    int64_t base;
    block_exclusive_scan<256>(above, s_wave, base);
    if (wave == 0) {
        const int64_t inc = wave_inclusive_scan(rt);
        if (lane < kSegDigits) s_row[lane] = (int32_t)(base + inc - rt + sp);
        if (total_out && seg == 0 && blockIdx.y == gridDim.y - 1 && lane == kSegDigits - 1) *total_out = base + inc;
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) s_block[2 * k + half][col] = t < tiles ? (int32_t)raw[k] : 0;
    __syncthreads();
    // Each wavefront scans 8 rows, two consecutive entries per lane.
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int r = wave * 8 + i;
        const int32_t a = s_block[r][2 * lane], b = s_block[r][2 * lane + 1];
        const int32_t ex = s_row[r] + wave_inclusive_scan(a + b) - (a + b);
        s_block[r][2 * lane] = ex;
        s_block[r][2 * lane + 1] = ex + a;
    }
    __syncthreads();
    const int dd = threadIdx.x & (kSegDigits - 1);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const int c = (threadIdx.x >> 5) + 8 * k;
        if (t0 + c < tiles) offsets[(t0 + c) * digits + d0 + dd] = s_block[dd][c];
    }
}

// Histogram and scan of one sort pass (digits of `bits` bits at `shift`;
// every key's digit below `digits`, a multiple of 32 up to R).
template <class K, int RB, bool DROP = false, int R = 1 << RB>
int sort_counts(const K* keys, int64_t count, int shift, uint32_t mask, int digits, const SortScratch& sc,
                hipStream_t s, const int64_t* live = nullptr, int64_t* total = nullptr,
                const uint32_t* key_base = nullptr);
inline int scan_counts(int64_t count, int digits, const SortScratch& sc, hipStream_t s, int64_t* total);

// tail_kind (1 or 2, 64-bit values only): the last pass also writes the
// order tail (record_extent<tail_kind>).
template <class K, class V = int32_t>
int run_sort(K* keys, V* values, int64_t count, int end_bit, void* scratch, hipStream_t s, int tail_kind = 0,
             OrderTail tail = OrderTail{}) {
    SortScratch sc;
    sort_scratch_bytes(count, &sc, scratch);
    const int64_t tiles = (count + kSortTile - 1) / kSortTile;
    K* kin = keys;
    V* vin = values;
    K* kout = keys + count;
    V* vout = values ? values + count : nullptr;
    for (int shift = 0; shift < end_bit; shift += 8) {
        const int bits = end_bit - shift < 8 ? end_bit - shift : 8;
        const uint32_t mask = (1u << bits) - 1u;
        const int status = sort_counts<K, 8>(kin, count, shift, mask, 256, sc, s);
        if (status != GS3D_OK) return status;
        const int tail_here = values && shift + 8 >= end_bit ? tail_kind : 0;
        if constexpr (sizeof(V) == 8) {
            if (tail_here == 1)
                hipLaunchKernelGGL((sort_scatter_kernel<K, V, true, 8, 1>), dim3((unsigned)tiles), dim3(kSortThreads),
                                   0, s, kin, vin, kout, vout, count, shift, mask, bits, sc.offsets, tiles, 256, tail,
                                   Culled{});
            else if (tail_here == 2)
                hipLaunchKernelGGL((sort_scatter_kernel<K, V, true, 8, 2>), dim3((unsigned)tiles), dim3(kSortThreads),
                                   0, s, kin, vin, kout, vout, count, shift, mask, bits, sc.offsets, tiles, 256, tail,
                                   Culled{});
        }
        if (tail_here == 0 || sizeof(V) != 8) {
            if (values)
                hipLaunchKernelGGL((sort_scatter_kernel<K, V, true>), dim3((unsigned)tiles), dim3(kSortThreads), 0, s,
                                   kin, vin, kout, vout, count, shift, mask, bits, sc.offsets, tiles, 256, OrderTail{},
                                   Culled{});
            else
                hipLaunchKernelGGL((sort_scatter_kernel<K, V, false>), dim3((unsigned)tiles), dim3(kSortThreads), 0, s,
                                   kin, vin, kout, vout, count, shift, mask, bits, sc.offsets, tiles, 256, OrderTail{},
                                   Culled{});
        }
        K* tk = kin;
        kin = kout;
        kout = tk;
        V* tv = vin;
        vin = vout;
        vout = tv;
    }
    if (kin != keys) {
        if (hipMemcpyAsync(keys, kin, (size_t)count * sizeof(K), hipMemcpyDeviceToDevice, s) != hipSuccess ||
            (values && hipMemcpyAsync(values, vin, (size_t)count * sizeof(V), hipMemcpyDeviceToDevice, s) != hipSuccess))
        {
            set_error("radix sort: copy of the sorted half failed");
            return GS3D_ERR_LAUNCH;
        }
    }
    return launch_status("radix sort");
}

// Passes of a depth order over key bits [0, end_bit), 9 <= end_bit <= 32:
// bits 0-7 first (the records kernel counts them), then 8-bit passes, the
// last one widened to up to 10 bits, so 25 or 26 key bits take three passes
// instead of four.  Returns the number of passes (2 to 4).
inline int order_passes(int end_bit, int (&shift)[4], int (&width)[4]) {
    int passes = 0, at = 0, rest = end_bit;
    shift[passes] = at;
    width[passes++] = 8;
    at += 8;
    rest -= 8;
    while (rest > 10) {
        shift[passes] = at;
        width[passes++] = 8;
        at += 8;
        rest -= 8;
    }
    shift[passes] = at;
    width[passes++] = rest;
    return passes;
}

// Radix bits of the order's count tables (its widest pass).
constexpr int kOrderRadixBits = 10;

// The depth order of the rows that touch a tile group: 32-bit keys with
// kDroppedKey for the others, 64-bit records, the passes of order_passes
// over bits [0, end_bit), the later ones of key - *key_base (key_base_kernel;
// null: of the key; every kept key minus the base must be below 2^end_bit).
// The first pass leaves the dropped rows out and its digit scan counts the rest
// into *live; the later passes sort [0, *live), and the last one writes
// `filler` records (and, with a tail, zero group counts) to [*live, count).
// The input is in the halves [start_half * count, ...) of keys and values,
// the half that leaves the result in the first halves after the passes:
// start_half = passes & 1.  Scratch: sort_scratch_bytes(count, ...,
// kOrderRadixBits).  tail_kind 0 or 1.
inline int run_order_sort(uint32_t* keys, uint64_t* values, int64_t count, void* scratch, int64_t* live,
                          uint64_t filler, hipStream_t s, int tail_kind, OrderTail tail, bool first_counted,
                          int end_bit, int start_half, const uint32_t* key_base) {
    SortScratch sc;
    sort_scratch_bytes(count, &sc, scratch, kOrderRadixBits);
    const int64_t tiles = (count + kSortTile - 1) / kSortTile;
    int shifts[4], widths[4];
    const int passes = order_passes(end_bit, shifts, widths);
    if (((passes + start_half) & 1) || tail_kind < 0 || tail_kind > 1) {
        set_error("depth order: input half or tail kind does not fit the passes");
        return GS3D_ERR_ARGUMENT;
    }
    uint32_t* kin = keys + start_half * count;
    uint64_t* vin = values + start_half * count;
    uint32_t* kout = keys + (1 - start_half) * count;
    uint64_t* vout = values + (1 - start_half) * count;
    const dim3 grid((unsigned)tiles), block(kSortThreads);
    for (int p = 0; p < passes; ++p) {
        const bool first = p == 0, last = p == passes - 1;
        const int shift = shifts[p], bits = widths[p];
        const uint32_t mask = (1u << bits) - 1u;
        const bool wide = bits > 8;
        const int digits = wide ? 1 << bits : 256;
        int status;
        if (first)
            status = first_counted ? scan_counts(count, 256, sc, s, live)
                                   : sort_counts<uint32_t, 8, true>(kin, count, shift, mask, 256, sc, s, nullptr, live);
        else if (wide && bits == 9)
            status = sort_counts<uint32_t, 9, false>(kin, count, shift, mask, digits, sc, s, live, nullptr, key_base);
        else if (wide)
            status = sort_counts<uint32_t, 10, false>(kin, count, shift, mask, digits, sc, s, live, nullptr, key_base);
        else
            status = sort_counts<uint32_t, 8, false>(kin, count, shift, mask, 256, sc, s, live, nullptr, key_base);
        if (status != GS3D_OK) return status;
        if (first) {
            hipLaunchKernelGGL((sort_scatter_kernel<uint32_t, uint64_t, true, 8, 0, true>), grid, block, 0, s, kin, vin,
                               kout, vout, count, shift, mask, bits, sc.offsets, tiles, 256, OrderTail{},
                               Culled{nullptr, false, 0});
        } else {
            const Culled cull{live, last, filler, key_base};
            const OrderTail t = last && tail_kind != 0 ? tail : OrderTail{};
            // Wide passes are compiled for their digit width (9 or 10 bits):
            // LDS counters and per-thread digit loops sized for it.
            if (wide && bits == 9 && last && tail_kind == 1)
                hipLaunchKernelGGL((sort_scatter_kernel<uint32_t, uint64_t, true, 9, 1>), grid, block, 0, s, kin, vin,
                                   kout, vout, count, shift, mask, bits, sc.offsets, tiles, digits, t, cull);
            else if (wide && bits == 9)
                hipLaunchKernelGGL((sort_scatter_kernel<uint32_t, uint64_t, true, 9, 0>), grid, block, 0, s, kin, vin,
                                   kout, vout, count, shift, mask, bits, sc.offsets, tiles, digits, t, cull);
            else if (wide && last && tail_kind == 1)
                hipLaunchKernelGGL((sort_scatter_kernel<uint32_t, uint64_t, true, 10, 1>), grid, block, 0, s, kin, vin,
                                   kout, vout, count, shift, mask, bits, sc.offsets, tiles, digits, t, cull);
            else if (wide)
                hipLaunchKernelGGL((sort_scatter_kernel<uint32_t, uint64_t, true, 10, 0>), grid, block, 0, s, kin, vin,
                                   kout, vout, count, shift, mask, bits, sc.offsets, tiles, digits, t, cull);
            else if (last && tail_kind == 1)
                hipLaunchKernelGGL((sort_scatter_kernel<uint32_t, uint64_t, true, 8, 1>), grid, block, 0, s, kin, vin,
                                   kout, vout, count, shift, mask, bits, sc.offsets, tiles, 256, t, cull);
            else
                hipLaunchKernelGGL((sort_scatter_kernel<uint32_t, uint64_t, true, 8, 0>), grid, block, 0, s, kin, vin,
                                   kout, vout, count, shift, mask, bits, sc.offsets, tiles, 256, t, cull);
        }
        std::swap(kin, kout);
        std::swap(vin, vout);
    }
    return launch_status("depth order");
}

// Histogram of TPB consecutive sort tiles per block: each digit's TPB counts
// are consecutive in the [digit][tile] layout, so a block writes runs of TPB
// 16-bit counts instead of one scattered count per digit.  One LDS histogram per tile
// (pitch R + 1: the transposed read is conflict-free).
// DROP and live as in sort_scatter_kernel (tiles at or beyond live count
// nothing, and their columns are written as zeros).  R as in
// sort_scatter_kernel.
template <class K, int RB, int TPB, bool DROP = false, int R = 1 << RB>
__global__ __launch_bounds__(kSortThreads) void sort_histogram_tiles_kernel(const K* __restrict__ keys, int64_t count,
                                                                            int shift, uint32_t mask,
                                                                            uint16_t* __restrict__ counts,
                                                                            int64_t tiles, int digits,
                                                                            const int64_t* __restrict__ live_count,
                                                                            const uint32_t* __restrict__ key_base) {
    static_assert(R <= (1 << RB), "digits of RB bits");
    constexpr int P = R + 1;
    const K base_key = key_base ? (K)*key_base : K(0);
    __shared__ uint32_t s_hist[TPB * P];
    for (int e = threadIdx.x; e < TPB * P; e += kSortThreads) s_hist[e] = 0;
    __syncthreads();
    const int64_t live = live_count ? min(count, *live_count) : count;
    const int64_t t0 = (int64_t)blockIdx.x * TPB;
    // The next tile's keys are loaded while this tile's are counted
    // (clamped addresses: no load waits behind a per-lane branch).
    auto load_tile = [&](int64_t base, K (&key)[kSortItems]) {
#pragma unroll
        for (int k = 0; k < kSortItems; ++k) key[k] = keys[min(base + k * kSortThreads + threadIdx.x, live - 1)];
    };
    K next[kSortItems];
    if (t0 * kSortTile < live) load_tile(t0 * kSortTile, next);
    for (int tt = 0; tt < TPB; ++tt) {
        const int64_t base = (t0 + tt) * kSortTile;
        if (base >= live) break;
        K key[kSortItems];
#pragma unroll
        for (int k = 0; k < kSortItems; ++k) key[k] = next[k];
        if (tt + 1 < TPB && base + kSortTile < live) load_tile(base + kSortTile, next);
#pragma unroll
        for (int k = 0; k < kSortItems; ++k) {
            const int64_t idx = base + k * kSortThreads + threadIdx.x;
            const bool valid = idx < live && !(DROP && key[k] == (K)kDroppedKey);
            const uint32_t d = digit_of((K)(key[k] - base_key), shift, mask);
            // A wavefront whose valid keys share one digit (high key bits:
            // exponents, view ids) adds them with one atomic instead of 64
            // serialised ones on the same LDS word.
            const uint64_t live = __ballot(valid);
            const uint32_t d0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)d);
            if (__ballot(valid && d != d0) == 0) {
                if (live && lane_id() == (int)__builtin_ctzll(live)) atomicAdd(&s_hist[tt * P + d0], (uint32_t)__popcll(live));
            } else if (valid) {
                atomicAdd(&s_hist[tt * P + d], 1u);
            }
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < TPB * digits; e += kSortThreads) {
        const int d = e / TPB, tt = e - d * TPB;
        const int64_t t = t0 + tt;
        if (t < tiles) counts[(int64_t)d * tiles + t] = (uint16_t)s_hist[tt * P + d];  // runs of TPB counts
    }
}

// Scan and transpose of a pass's [digit][tile] counts (already in sc.counts).
inline int scan_counts(int64_t count, int digits, const SortScratch& sc, hipStream_t s, int64_t* total) {
    const int64_t tiles = (count + kSortTile - 1) / kSortTile;
    if (tiles * digits <= kSingleScanMax) {
        // Small table: scanned and written transposed by one workgroup.
        hipLaunchKernelGGL((scan_single_kernel<uint16_t, false>), dim3(1), dim3(kSingleThreads), 0, s, sc.counts,
                           tiles * digits, sc.offsets, total, (int32_t)tiles, (int32_t)digits, SideSum{});
        return launch_status("radix sort counts");
    }
    const int64_t segs = (tiles + kSegTiles - 1) / kSegTiles;
    int32_t* seg_prefix = sc.scan;
    int32_t* row_totals = sc.scan + segs * digits;
    // The fewest words a thread (a multiple of 8, at most 48) that cover a
    // row in one chunk; longer rows loop over chunks of 48.
    launch_digit_rows<8>((int)((tiles + kRowThreads - 1) / kRowThreads), digits, sc.counts, (int)tiles, (int)segs,
                         seg_prefix, row_totals, s);
    hipLaunchKernelGGL(digit_offsets_kernel, dim3((unsigned)segs, digits / kSegDigits), dim3(256), 0, s, sc.counts,
                       tiles, digits, seg_prefix, row_totals, sc.offsets, total);
    return launch_status("radix sort counts");
}

// total (optional) receives the number of keys counted.
template <class K, int RB, bool DROP, int R>
int sort_counts(const K* keys, int64_t count, int shift, uint32_t mask, int digits, const SortScratch& sc,
                hipStream_t s, const int64_t* live, int64_t* total, const uint32_t* key_base) {
    // Tiles per histogram block (the length of each digit's run of counts):
    // GS3D_HIST_TILES8 for 8-bit digits, 8 for wider ones.
    constexpr int TPB = RB > 8 ? 8 : GS3D_HIST_TILES8;
    const int64_t tiles = (count + kSortTile - 1) / kSortTile;
    hipLaunchKernelGGL((sort_histogram_tiles_kernel<K, RB, TPB, DROP, R>), dim3((unsigned)((tiles + TPB - 1) / TPB)),
                       dim3(kSortThreads), 0, s, keys, count, shift, mask, sc.counts, tiles, digits, live, key_base);
    return scan_counts(count, digits, sc, s, total);
}

// Start and end of every digit's run in the output of a one-pass sort: row
// 0 of the transposed offsets holds each digit's start.
__global__ void digit_ranges_kernel(const int32_t* __restrict__ offsets, int64_t count, int digits,
                                    int ranges_count, int32_t* __restrict__ ranges) {
    const int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= ranges_count) return;
    const int32_t start = offsets[d];
    const int32_t end = d + 1 < digits ? offsets[d + 1] : (int32_t)count;
    ranges[2 * d] = start;
    ranges[2 * d + 1] = end;
}

// Everything the group passes need from a one-pass group sort, in one
// workgroup (groups <= 1024): each group's range of sorted items (row 0 of
// the transposed offsets holds every digit's start), chunk_base (exclusive
// scan of the groups' chunk counts, the chunk total at [groups]) and the
// group of every chunk.  One launch instead of three latency-bound ones.
constexpr int kChunkSteps = 8;  // items per lane of a group chunk (4 and 16 measured slower)
constexpr int kChunk = 64 * kChunkSteps;  // items of a group ranked by one wavefront
constexpr int kLayoutThreads = 1024;

__global__ __launch_bounds__(kLayoutThreads) void group_layout_kernel(const int32_t* __restrict__ offsets,
                                                                      int64_t count, int digits, int groups,
                                                                      int32_t* __restrict__ ranges,
                                                                      int32_t* __restrict__ chunk_base,
                                                                      int32_t* __restrict__ chunk_group) {
    __shared__ int32_t s_wave[kLayoutThreads / 64];
    __shared__ int32_t s_base[kLayoutThreads + 1];
    const int g = threadIdx.x;
    int32_t q = 0;
    if (g < groups) {
        const int32_t start = offsets[g];
        const int32_t end = g + 1 < digits ? offsets[g + 1] : (int32_t)count;
        ranges[2 * g] = start;
        ranges[2 * g + 1] = end;
        q = (end - start + kChunk - 1) / kChunk;
    }
    int32_t total;
    const int32_t ex = block_exclusive_scan<kLayoutThreads>(q, s_wave, total);
    if (g < groups) {
        chunk_base[g] = ex;
        s_base[g] = ex;
    }
    if (g == 0) {
        chunk_base[groups] = total;
        s_base[groups] = total;
    }
    __syncthreads();
    // Wavefront w writes the chunk entries of groups w, w + 16, ...
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    for (int h = wave; h < groups; h += kLayoutThreads / 64) {
        const int32_t end = s_base[h + 1];
        for (int32_t u = s_base[h] + lane; u < end; u += 64) chunk_group[u] = h;
    }
}

// Stable keys-only sort of keys[0:count) on bits [0, end_bit), end_bit <=
// kOnePassBits, in one 10-bit pass: the result is written to
// keys[count:2count) and ranges[2d], ranges[2d + 1] (d < ranges_count)
// receive the run of key value d.  With chunk_base, the group layout of
// group_layout_kernel is written too (ranges_count groups, at most 1024).
// Scratch as sort_scratch_bytes(count, ..., kOnePassBits).
constexpr int kOnePassBits = 10;

template <class K>
int run_sort_once(K* keys, int64_t count, int end_bit, void* scratch, int ranges_count, int32_t* ranges,
                  hipStream_t s, int32_t* chunk_base = nullptr, int32_t* chunk_group = nullptr) {
    constexpr int RB = kOnePassBits;
    SortScratch sc;
    sort_scratch_bytes(count, &sc, scratch, RB);
    const int64_t tiles = (count + kSortTile - 1) / kSortTile;
    const uint32_t mask = (1u << end_bit) - 1u;
    // Only the digits of the key range are counted, scanned and transposed
    // (the keys are below ranges_count).
    const int digits = min(1 << RB, (ranges_count + 31) & ~31);
    // Up to 768 key values the histogram and scatter keep 768 LDS counters
    // per row instead of 1024 (the keys are below ranges_count <= digits).
    auto sort_pass = [&](auto counters) -> int {
        constexpr int R = decltype(counters)::value;
        const int status = sort_counts<K, RB, false, R>(keys, count, 0, mask, digits, sc, s);
        if (status != GS3D_OK) return status;
        hipLaunchKernelGGL((sort_scatter_kernel<K, int32_t, false, RB, 0, false, R>), dim3((unsigned)tiles),
                           dim3(kSortThreads), 0, s, keys, (const int32_t*)nullptr, keys + count, (int32_t*)nullptr,
                           count, 0, mask, end_bit, sc.offsets, tiles, digits, OrderTail{}, Culled{});
        return GS3D_OK;
    };
    const int status = digits <= 768 ? sort_pass(std::integral_constant<int, 768>{})
                                     : sort_pass(std::integral_constant<int, 1 << RB>{});
    if (status != GS3D_OK) return status;
    if (chunk_base)
        hipLaunchKernelGGL(group_layout_kernel, dim3(1), dim3(kLayoutThreads), 0, s, sc.offsets, count, digits,
                           ranges_count, ranges, chunk_base, chunk_group);
    else
        hipLaunchKernelGGL(digit_ranges_kernel, dim3((unsigned)((ranges_count + 255) / 256)), dim3(256), 0, s,
                           sc.offsets, count, digits, ranges_count, ranges);
    return launch_status("one-pass radix sort");
}

// ---------------------------------------------------------------------------
// Per-tile ranges (primitives/tiling.py:39-54).  Tile ids at or beyond
// tile_count (0xFFFFFFFF included) are ignored.
// ---------------------------------------------------------------------------
template <class K>
__global__ void tile_ranges_kernel(const K* __restrict__ keys, int64_t count, int shift, uint32_t mask,
                                   int32_t* __restrict__ ranges, int64_t tile_count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const int64_t cur = (int64_t)((uint32_t)(keys[i] >> shift) & mask);
    const bool cur_ok = cur < tile_count;
    if (i == 0) {
        if (cur_ok) ranges[2 * cur] = 0;
    } else {
        const int64_t prev = (int64_t)((uint32_t)(keys[i - 1] >> shift) & mask);
        if (cur != prev) {
            if (prev < tile_count) ranges[2 * prev + 1] = (int32_t)i;
            if (cur_ok) ranges[2 * cur] = (int32_t)i;
        }
    }
    if (i == count - 1 && cur_ok) ranges[2 * cur + 1] = (int32_t)count;
}

// ---------------------------------------------------------------------------
// Grouped binning.  Every tile's list holds, in (depth bits, Gaussian index)
// order, the Gaussians whose tile rectangle covers it; lists are laid out in
// global tile order.  That is the order of a stable sort of the reference's
// (tile << 32 | depth bits) keys over Gaussian-ordered pairs
// (splatting/binning.py:16-37, primitives/tiling.py:67-100), produced here
// without sorting the pairs:
//   * rows (view, Gaussian) are stably sorted by depth bits;
//   * each row yields one item per 8x8-tile group its rectangle touches
//     (group id, the rectangle clipped to the group, the Gaussian index),
//     emitted in depth order and stably sorted by group (a short radix sort:
//     groups number in the hundreds);
//   * a group's item list is cut into 512-item chunks, one per wavefront.
//     Lane t of the wavefront owns tile t of the group: for every tile that
//     some item of a 64-item step touches, a ballot gives each item its rank
//     among the step's items on that tile, and lane t keeps the running
//     count.  A counting pass stores each chunk's per-tile counts, one
//     exclusive scan turns them into per-(tile, chunk) offsets and tile
//     totals, a scan of the totals gives tile starts, and the writing pass
//     stores every Gaussian index straight to its final position.
// ---------------------------------------------------------------------------
constexpr int kGroupShift = 3;  // groups of 8x8 tiles: one wavefront lane per tile
constexpr int kGroupBits = 20;  // group id field (low bits) of an item
constexpr uint32_t kGroupMask = (1u << kGroupBits) - 1u;
constexpr int kBinThreads = 256;
constexpr int kBinWaves = kBinThreads / 64;

struct GridDims {
    int gx, gy, tpv;   // tiles per row, per column, per view
    int sgx, sgy, gpv; // groups per row, per column, per view
};

inline GridDims grid_dims(int width, int height) {
    GridDims d;
    d.gx = (width + 15) / 16;
    d.gy = (height + 15) / 16;
    d.tpv = d.gx * d.gy;
    d.sgx = (d.gx + 7) >> kGroupShift;
    d.sgy = (d.gy + 7) >> kGroupShift;
    d.gpv = d.sgx * d.sgy;
    return d;
}

GS3D_DEV uint64_t pack_rect(int x0, int y0, int x1, int y1) {
    return (uint64_t)(uint32_t)x0 | ((uint64_t)(uint32_t)y0 << 16) | ((uint64_t)(uint32_t)x1 << 32) |
           ((uint64_t)(uint32_t)y1 << 48);
}

// Bit (ly*8 + lx) set for every tile of the clipped rectangle
// [lx0, lx1] x [ly0, ly1] (inclusive, 3 bits each, packed lx0 | lx1 << 3 |
// ly0 << 6 | ly1 << 9).
GS3D_DEV uint64_t group_tile_mask(uint32_t local) {
    const int lx0 = local & 7, lx1 = (local >> 3) & 7, ly0 = (local >> 6) & 7, ly1 = (local >> 9) & 7;
    const uint64_t row = (2ull << lx1) - (1ull << lx0);
    const uint64_t rows = (~0ull >> (8 * (7 - ly1))) & (~0ull << (8 * ly0));
    return (row * 0x0101010101010101ull) & rows;
}

GS3D_DEV uint64_t wave_or64(uint64_t v) {
    uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        lo |= (uint32_t)__shfl_xor((int)lo, d, 64);
        hi |= (uint32_t)__shfl_xor((int)hi, d, 64);
    }
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)hi) << 32) |
           (uint32_t)__builtin_amdgcn_readfirstlane((int)lo);
}

// Ordered row records: row index in the low 32 bits; for tile grids of at
// most 256 x 256 the high 32 bits carry the row's tile rectangle
// (x0 | y0 << 8 | (x1 - 1) << 16 | (y1 - 1) << 24, kEmptyRect for culled
// rows) so that nothing downstream gathers per-row data in depth order.
// Larger grids leave the high half zero and recompute the rectangle from the
// row's centre and radius.
constexpr uint32_t kEmptyRect = 0x000000FFu;  // x0 = 255 > x1 - 1 = 0

struct TileRect {
    int x0, y0, x1, y1;  // exclusive ends; empty when x1 <= x0
};

// Per-row inputs of the tile footprint (conics are read only outside the
// radius mode).
struct RowGeometry {
    const float* centers;
    const float* conics;
    const int32_t* radii;
    int mode;
};

GS3D_DEV TileRect rect_of(int radius, float2 c, float4 k, int gx, int gy, int mode) {
    TileRect r{0, 0, 0, 0};
    if (radius > 0) {
        const int4 b = mode_rect(c, k, radius, gx, gy, mode);
        if (b.z > b.x && b.w > b.y) r = TileRect{b.x, b.y, b.z, b.w};
    }
    return r;
}

GS3D_DEV TileRect row_rect(const RowGeometry& g, int64_t row, int gx, int gy) {
    // Centre and conic are loaded with the radius, not after it.
    const int radius = g.radii[row];
    const float2 c = reinterpret_cast<const float2*>(g.centers)[row];
    const float4 k = g.mode == GS3D_TILE_RADIUS ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
                                                : reinterpret_cast<const float4*>(g.conics)[row];
    asm volatile("" ::"v"(c.x), "v"(c.y), "v"(k.x), "v"(k.y), "v"(k.z), "v"(k.w));
    return rect_of(radius, c, k, gx, gy, g.mode);
}

template <bool PACKED>
GS3D_DEV TileRect record_rect(uint64_t record, const RowGeometry& g, int gx, int gy) {
    if constexpr (PACKED) {
        const uint32_t p = (uint32_t)(record >> 32);
        TileRect r{(int)(p & 255u), (int)((p >> 8) & 255u), (int)((p >> 16) & 255u) + 1, (int)(p >> 24) + 1};
        if (r.x1 <= r.x0) r = TileRect{0, 0, 0, 0};
        return r;
    } else {
        return row_rect(g, (int64_t)(uint32_t)record, gx, gy);
    }
}

// AccuTile groups and tiles of one footprint.  Strips of one group row (8
// strips) touch an interval of group columns: consecutive strips share the
// crossing points of their common boundary line, so their tile spans
// overlap and the union over the group row is one interval.  Emission uses
// the same intervals, so counts and items always agree.
GS3D_DEV void accutile_groups(const Ellipse& e, int& groups, int& tiles) {
    bool is_y = true;
    int cur = -1, gmin = INT_MAX, gmax = -1, total = 0;
    tiles = accutile_strips(e, is_y, [&](int row, int lo, int hi) {
        const int G = row >> kGroupShift;
        if (G != cur) {
            if (gmax >= gmin) total += gmax - gmin + 1;
            cur = G;
            gmin = INT_MAX;
            gmax = -1;
        }
        if (hi > lo) {
            gmin = min(gmin, lo >> kGroupShift);
            gmax = max(gmax, (hi - 1) >> kGroupShift);
        }
    });
    if (gmax >= gmin) total += gmax - gmin + 1;
    groups = total;
}

GS3D_DEV int groups_of(const TileRect& r) {
    if (r.x1 <= r.x0) return 0;
    return (((r.x1 - 1) >> kGroupShift) - (r.x0 >> kGroupShift) + 1) *
           (((r.y1 - 1) >> kGroupShift) - (r.y0 >> kGroupShift) + 1);
}

// Group count and tile pairs of a packed record (the order tail; the same
// values order_counts_kernel computes for PACKED records).
template <int TAIL>
GS3D_DEV void record_extent(uint64_t record, int32_t& groups, int64_t& area) {
    if constexpr (TAIL == 1) {
        const TileRect r = record_rect<true>(record, RowGeometry{nullptr, nullptr, nullptr, 0}, 0, 0);
        groups = groups_of(r);
        area = r.x1 > r.x0 ? (int64_t)(r.x1 - r.x0) * (r.y1 - r.y0) : 0;
    } else {
        const uint32_t hi = (uint32_t)(record >> 32);
        groups = (int32_t)(hi & 4095u);
        area = hi >> 12;
    }
}

// Row order under AccuTile: depth-bit keys and records (coalesced reads of
// depth, centre and radius).  The row's footprint and strips are computed
// here, once, in row order; on grids of at most 256 x 256 tiles the record's
// high half carries tiles << 12 | groups and footprints[row] the compact
// footprint, so the depth-ordered passes neither gather nor recompute it.
// tiles_out (optional) receives every row's tile count in the mode.
template <bool PACKED>
__global__ void row_records_kernel(const float* __restrict__ depths, RowGeometry g, int64_t rows, int gx, int gy,
                                   uint32_t* __restrict__ keys, uint64_t* __restrict__ records,
                                   int32_t* __restrict__ tiles_out, float4* __restrict__ footprints) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows) return;
    uint64_t rec = (uint64_t)(uint32_t)i;
    int groups = 0, tiles = 0;
    const int radius = g.radii[i];
    if (radius > 0) {
        const Ellipse e = footprint(reinterpret_cast<const float2*>(g.centers)[i],
                                    reinterpret_cast<const float4*>(g.conics)[i], radius, gx, gy);
        accutile_groups(e, groups, tiles);
        if constexpr (PACKED) {
            float4 p0, p1;
            pack_ellipse(e, p0, p1);
            footprints[2 * i] = p0;
            footprints[2 * i + 1] = p1;
        }
    }
    if constexpr (PACKED) rec |= (uint64_t)(((uint32_t)tiles << 12) | (uint32_t)groups) << 32;
    if (tiles_out) tiles_out[i] = tiles;
    keys[i] = __float_as_uint(depths[i]);
    records[i] = rec;
}

// Row order outside AccuTile: depth-bit keys and records, rows whose
// footprint touches no tile keyed kDroppedKey (the depth order leaves them
// out); record high halves as in the packed layout above.  One 2048-row sort
// tile per block, which also counts the tile's keys by bits 0-7 for the depth
// order's first pass (dropped rows not counted): the [digit][tile] table that
// pass's histogram would form, without reading the keys again; and writes the
// smallest and largest kept key of the tile to block_range[2 * tile + {0, 1}]
// (0xFFFFFFFF, 0 when it keeps none).  Every load of a thread's eight rows is
// issued first (clamped to the last row).
template <bool PACKED>
__global__ __launch_bounds__(kSortThreads) void row_records_counted_kernel(
    const float* __restrict__ depths, RowGeometry g, int64_t rows, int gx, int gy, uint32_t* __restrict__ keys,
    uint64_t* __restrict__ records, int32_t* __restrict__ tiles_out, uint16_t* __restrict__ counts, int64_t tiles,
    uint32_t* __restrict__ block_range) {
    static_assert(kSortThreads == kRadix, "one digit per thread");
    __shared__ uint32_t s_hist[kRadix];
    __shared__ uint32_t s_range[2];
    s_hist[threadIdx.x] = 0u;
    if (threadIdx.x == 0) {
        s_range[0] = 0xFFFFFFFFu;
        s_range[1] = 0u;
    }
    const int64_t tile = xcd_contiguous(blockIdx.x, gridDim.x);
    const int64_t base = tile * kSortTile + threadIdx.x;
    float dep[kSortItems];
    int rad[kSortItems];
    float2 cen[kSortItems];
    float4 con[kSortItems];
#pragma unroll
    for (int k = 0; k < kSortItems; ++k) {
        const int64_t i = min(base + k * kSortThreads, rows - 1);
        dep[k] = depths[i];
        rad[k] = g.radii[i];
        cen[k] = reinterpret_cast<const float2*>(g.centers)[i];
        con[k] = g.mode == GS3D_TILE_RADIUS ? make_float4(0.0f, 0.0f, 0.0f, 0.0f)
                                            : reinterpret_cast<const float4*>(g.conics)[i];
    }
    __syncthreads();
    uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
#pragma unroll
    for (int k = 0; k < kSortItems; ++k) {
        const int64_t i = base + k * kSortThreads;
        if (i >= rows) continue;
        const TileRect r = rect_of(rad[k], cen[k], con[k], gx, gy, g.mode);
        uint64_t rec = (uint64_t)(uint32_t)i;
        if constexpr (PACKED) {
            const uint32_t p = r.x1 > r.x0 ? (uint32_t)r.x0 | ((uint32_t)r.y0 << 8) |
                                                 ((uint32_t)(r.x1 - 1) << 16) | ((uint32_t)(r.y1 - 1) << 24)
                                           : kEmptyRect;
            rec |= (uint64_t)p << 32;
        }
        if (tiles_out) tiles_out[i] = r.x1 > r.x0 ? (r.x1 - r.x0) * (r.y1 - r.y0) : 0;
        const uint32_t key = r.x1 > r.x0 ? __float_as_uint(dep[k]) : kDroppedKey;
        keys[i] = key;
        records[i] = rec;
        if (key != kDroppedKey) {
            atomicAdd(&s_hist[key & 255u], 1u);
            kmin = min(kmin, key);
            kmax = max(kmax, key);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, o));
        kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o));
    }
    if (lane_id() == 0) {
        atomicMin(&s_range[0], kmin);
        atomicMax(&s_range[1], kmax);
    }
    __syncthreads();
    counts[(int64_t)threadIdx.x * tiles + tile] = (uint16_t)s_hist[threadIdx.x];
    if (threadIdx.x == 0) {
        block_range[2 * tile] = s_range[0];
        block_range[2 * tile + 1] = s_range[1];
    }
}

// Group count of every row in depth order; the block's tile pair count goes
// to block_pairs[blockIdx.x].  ACCU: AccuTile strips of the row's footprint.
// live (optional): ordered rows at or beyond *live are fillers with no groups.
template <bool PACKED, bool ACCU>
__global__ __launch_bounds__(kBinThreads) void order_counts_kernel(const uint64_t* __restrict__ records, int64_t rows,
                                                                   RowGeometry g, int gx, int gy,
                                                                   int32_t* __restrict__ group_counts,
                                                                   int64_t* __restrict__ block_pairs,
                                                                   const int64_t* __restrict__ live) {
    __shared__ int64_t s_wave[kBinWaves];
    const int64_t i = (int64_t)blockIdx.x * kBinThreads + threadIdx.x;
    int64_t area = 0;
    if (live && i >= *live && i < rows) {
        group_counts[i] = 0;
    } else if (i < rows) {
        if constexpr (ACCU && PACKED) {
            const uint32_t hi = (uint32_t)(records[i] >> 32);
            area = hi >> 12;
            group_counts[i] = (int32_t)(hi & 4095u);
        } else if constexpr (ACCU) {
            const int64_t row = (int64_t)(uint32_t)records[i];
            const int radius = g.radii[row];
            int groups = 0, tiles = 0;
            if (radius > 0)
                accutile_groups(footprint(reinterpret_cast<const float2*>(g.centers)[row],
                                          reinterpret_cast<const float4*>(g.conics)[row], radius, gx, gy),
                                groups, tiles);
            area = tiles;
            group_counts[i] = groups;
        } else {
            const TileRect r = record_rect<PACKED>(records[i], g, gx, gy);
            if (r.x1 > r.x0) area = (int64_t)(r.x1 - r.x0) * (r.y1 - r.y0);
            group_counts[i] = groups_of(r);
        }
    }
    int64_t total;
    block_exclusive_scan<kBinThreads>(area, s_wave, total);
    if (threadIdx.x == 0) block_pairs[blockIdx.x] = total;
}

// Base of the depth order's later passes (one block): the smallest kept key
// of all sort tiles (block_range pairs from row_records_counted_kernel) with
// its low byte cleared.  Those passes take their digits from key - *base,
// whose low byte is the key's own, so the first pass (counted on raw low
// bytes) and the later ones sort the same numbers, and the differences may
// need fewer bits than the keys (depths on both sides of a power of two).
// key_bits (optional) receives the bits the largest difference needs, 0
// without kept keys; without block_range (orders that sort raw 32-bit keys)
// it receives 32 and *base is left alone.
__global__ __launch_bounds__(1024) void key_base_kernel(const uint32_t* __restrict__ block_range, int64_t ranges,
                                                        uint32_t* __restrict__ base, int32_t* __restrict__ key_bits) {
    __shared__ uint32_t s_range[2];
    if (!block_range) {
        if (key_bits && threadIdx.x == 0) *key_bits = 32;
        return;
    }
    if (threadIdx.x == 0) {
        s_range[0] = 0xFFFFFFFFu;
        s_range[1] = 0u;
    }
    __syncthreads();
    uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
    for (int64_t i = threadIdx.x; i < ranges; i += 1024) {
        kmin = min(kmin, block_range[2 * i]);
        kmax = max(kmax, block_range[2 * i + 1]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, o));
        kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o));
    }
    if (lane_id() == 0) {
        atomicMin(&s_range[0], kmin);
        atomicMax(&s_range[1], kmax);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t lo = s_range[0], hi = s_range[1];
        const bool any = lo <= hi;
        const uint32_t b = any ? lo & ~255u : 0u;
        *base = b;
        if (key_bits) *key_bits = any ? 32 - __clz((int)(hi - b)) : 0;
    }
}

// One block per 256 ordered rows; the block's items form one contiguous
// output range, filled with stride 256 (coalesced), each item locating its
// row by binary search over the rows' inclusive ends in LDS.
// Item = Gaussian index << 32 | clipped rectangle << 20 | group id.
constexpr int kEmitOwners = 2048;
static_assert(kBinThreads <= 256, "owner map entries are bytes");

template <bool PACKED>
__global__ __launch_bounds__(kBinThreads) void group_emit_kernel(const uint64_t* __restrict__ records,
                                                                 const int32_t* __restrict__ offsets, int64_t rows,
                                                                 RowGeometry geo, int n, GridDims d,
                                                                 int64_t limit, uint64_t* __restrict__ items) {
    __shared__ int32_t s_end[kBinThreads];
    __shared__ int32_t s_x0[kBinThreads], s_y0[kBinThreads], s_x1[kBinThreads], s_y1[kBinThreads];
    __shared__ int32_t s_gw[kBinThreads];
    __shared__ uint32_t s_gbase[kBinThreads];
    __shared__ uint32_t s_id[kBinThreads];
    __shared__ uint8_t s_owner[kEmitOwners];
    const int64_t r0 = (int64_t)blockIdx.x * kBinThreads;
    const int cnt = (int)min((int64_t)kBinThreads, rows - r0);
    const int t = threadIdx.x;
    const int64_t S = r0 > 0 ? offsets[r0 - 1] : 0;  // issued with the rows' loads
    if (t < cnt) {
        const int64_t i = r0 + t;
        const uint64_t rec = records[i];
        const int32_t end = offsets[i];
        asm volatile("" ::"v"(end));  // loaded beside the record, not after its decoding
        const int32_t row = (int32_t)(uint32_t)rec;
        const TileRect r = record_rect<PACKED>(rec, geo, d.gx, d.gy);
        s_end[t] = end;
        s_x0[t] = r.x0;
        s_y0[t] = r.y0;
        s_x1[t] = r.x1;
        s_y1[t] = r.y1;
        s_gw[t] = r.x1 > r.x0 ? ((r.x1 - 1) >> kGroupShift) - (r.x0 >> kGroupShift) + 1 : 1;
        const int view = row / n;
        s_gbase[t] = (uint32_t)(view * d.gpv);
        s_id[t] = (uint32_t)(row - view * n);
    }
    __syncthreads();
    const int64_t E = min((int64_t)s_end[cnt - 1], limit);
    // Blocks of at most kEmitOwners items look their rows up in an owner map
    // that the rows fill (one byte per item); larger ones search.
    const bool mapped = (int64_t)s_end[cnt - 1] - S <= kEmitOwners;
    if (mapped) {
        if (t < cnt) {
            const int32_t from = (t > 0 ? s_end[t - 1] : (int32_t)S) - (int32_t)S, to = s_end[t] - (int32_t)S;
            for (int32_t q = from; q < to; ++q) s_owner[q] = (uint8_t)t;
        }
        __syncthreads();
    }
    for (int64_t p = S + t; p < E; p += kBinThreads) {
        int lo = 0;
        if (mapped) {
            lo = s_owner[p - S];
        } else {
            // First j with s_end[j] > p (p < s_end[cnt - 1], offsets are
            // int32): a fixed 8-step search, every entry below lo ends at or
            // before p.
            const int32_t p32 = (int32_t)p;
#pragma unroll
            for (int step = kBinThreads / 2; step > 0; step >>= 1)
                if (lo + step <= cnt && s_end[lo + step - 1] <= p32) lo += step;
        }
        const int64_t start = lo > 0 ? s_end[lo - 1] : S;
        const int local = (int)(p - start);
        const int gw = s_gw[lo];
        int oy;
        if constexpr (PACKED) {
            // local < gw * gh <= 32 * 32: (local + 0.5) / gw is at least
            // 0.5 / gw >= 1/64 away from an integer, far beyond the
            // reciprocal's error, so truncation gives the exact quotient.
            oy = (int)(((float)local + 0.5f) * __builtin_amdgcn_rcpf((float)gw));
        } else {
            oy = local / gw;
        }
        const int ox = local - oy * gw;
        const int X = (s_x0[lo] >> kGroupShift) + ox, Y = (s_y0[lo] >> kGroupShift) + oy;
        const int lx0 = max(s_x0[lo] - (X << kGroupShift), 0), lx1 = min(s_x1[lo] - 1 - (X << kGroupShift), 7);
        const int ly0 = max(s_y0[lo] - (Y << kGroupShift), 0), ly1 = min(s_y1[lo] - 1 - (Y << kGroupShift), 7);
        const uint32_t gid = s_gbase[lo] + (uint32_t)(Y * d.sgx + X);
        const uint32_t clip = (uint32_t)(lx0 | (lx1 << 3) | (ly0 << 6) | (ly1 << 9));
        st_stream(items + p, ((uint64_t)s_id[lo] << 32) | ((uint64_t)clip << kGroupBits) | gid);
    }
}

// AccuTile items: one thread per ordered row writes one item per group of
// each group row's interval (accutile_groups), with the 64-bit mask of the
// group's tiles its strips cover (bit ly * 8 + lx), in masks[].  The spans
// of the current group row's 8 strips wait in per-thread LDS slots.
// PACKED: footprints come from the compact per-row copies written by
// row_records_kernel (one 32-byte gather), else they are recomputed.
// Rows whose footprint spans more strips than this are emitted by their
// whole wavefront (one group-row of 8 strips per lane), the others by one
// thread each.
constexpr int kCoopStrips = 16;

// The 64-bit tile mask of group column gc of a group-row, from its 8 strip
// spans (tile intervals along the strips' long direction).
GS3D_DEV uint64_t group_mask(const int2 (&span)[1 << kGroupShift], int gc, bool is_y) {
    const int c0 = gc << kGroupShift;
    uint64_t m = 0;
#pragma unroll
    for (int j = 0; j < (1 << kGroupShift); ++j) {
        const int lo = max(span[j].x, c0), hi = min(span[j].y, c0 + 8);
        if (hi <= lo) continue;
        if (is_y) {
            m |= (((1ull << (hi - lo)) - 1ull) << (lo - c0)) << (8 * j);
        } else {
            // column strip j: bit 8 * (k - c0) + j for k in [lo, hi)
            const uint64_t bytes = (hi - c0 == 8 ? ~0ull : (1ull << (8 * (hi - c0))) - 1ull) & ~((1ull << (8 * (lo - c0))) - 1ull);
            m |= (0x0101010101010101ull & bytes) << j;
        }
    }
    return m;
}

// Items of one row in group-row order, then group-column order, at
// [start, stop): rows spanning few strips by their own thread, the others by
// their whole wavefront (lanes take group-rows; a wave prefix sum of the
// lanes' item counts gives each group-row's place, so the items land exactly
// where the one-thread walk puts them).
template <bool PACKED>
__global__ __launch_bounds__(kBinThreads) void accutile_emit_kernel(const uint64_t* __restrict__ records,
                                                                    const int32_t* __restrict__ offsets, int64_t rows,
                                                                    RowGeometry geo, const float4* __restrict__ footprints,
                                                                    int n, GridDims d, int64_t limit,
                                                                    uint64_t* __restrict__ items,
                                                                    uint64_t* __restrict__ masks) {
    __shared__ int2 s_span[1 << kGroupShift][kBinThreads];
    const int t = threadIdx.x;
    const int lane = lane_id();
    const int64_t i = (int64_t)blockIdx.x * kBinThreads + t;
    int64_t start = 0, stop = 0, row = 0;
    float4 p0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), p1 = p0, conic = p0;
    float2 center = make_float2(0.0f, 0.0f);
    int radius = 0;
    bool live = false;
    if (i < rows) {
        start = i > 0 ? offsets[i - 1] : 0;
        stop = min((int64_t)offsets[i], limit);
        if (start < stop) {
            row = (int64_t)(uint32_t)records[i];
            if constexpr (PACKED) {
                p0 = footprints[2 * row];
                p1 = footprints[2 * row + 1];
                live = true;
            } else {
                radius = geo.radii[row];
                if (radius > 0) {
                    center = reinterpret_cast<const float2*>(geo.centers)[row];
                    conic = reinterpret_cast<const float4*>(geo.conics)[row];
                    live = true;
                }
            }
        }
    }
    auto ellipse_of = [&](float4 q0, float4 q1, float2 ctr, float4 con, int rad) {
        if constexpr (PACKED)
            return unpack_ellipse(q0, q1);
        else
            return footprint(ctr, con, rad, d.gx, d.gy);
    };
    int strips = 0;
    Ellipse e{};
    if (live) {
        e = ellipse_of(p0, p1, center, conic, radius);
        const int nx = max(0, e.bounds.z - e.bounds.x), ny = max(0, e.bounds.w - e.bounds.y);
        strips = (nx == 0 || ny == 0) ? 0 : min(nx, ny);
    }
    const bool coop = strips > kCoopStrips;
    if (live && !coop) {
        const int view = (int)(row / n);
        const uint64_t id = (uint64_t)(uint32_t)(row - (int64_t)view * n);
        const uint32_t gbase = (uint32_t)(view * d.gpv);
        int64_t p = start;
        bool is_y = true;
        int cur = -1, gmin = INT_MAX, gmax = -1;
        auto flush = [&](int G) {
            int2 span[1 << kGroupShift];
#pragma unroll
            for (int j = 0; j < (1 << kGroupShift); ++j) span[j] = s_span[j][t];
            for (int gc = gmin; gc <= gmax; ++gc) {
                const uint64_t m = group_mask(span, gc, is_y);
                const int GX = is_y ? gc : G, GY = is_y ? G : gc;
                if (p < stop) {
                    st_stream(items + p, (id << 32) | (uint64_t)(gbase + (uint32_t)(GY * d.sgx + GX)));
                    st_stream(masks + p, m);
                }
                ++p;
            }
        };
        accutile_strips(e, is_y, [&](int strip, int lo, int hi) {
            const int G = strip >> kGroupShift;
            if (G != cur) {
                if (cur >= 0) flush(cur);
                cur = G;
                gmin = INT_MAX;
                gmax = -1;
                for (int j = 0; j < (1 << kGroupShift); ++j) s_span[j][t] = make_int2(0, 0);
            }
            s_span[strip & 7][t] = make_int2(lo, hi);
            if (hi > lo) {
                gmin = min(gmin, lo >> kGroupShift);
                gmax = max(gmax, (hi - 1) >> kGroupShift);
            }
        });
        if (cur >= 0) flush(cur);
    }
    // Wide rows: the wavefront takes them one at a time.
    uint64_t todo = __ballot(coop);
    while (todo) {
        const int src = __builtin_ctzll(todo);
        todo &= todo - 1;
        auto bcast_f = [&](float v) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src)); };
        auto bcast_i64 = [&](int64_t v) {
            const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, src);
            const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), src);
            return (int64_t)(((uint64_t)hi << 32) | lo);
        };
        const int64_t w_start = bcast_i64(start), w_stop = bcast_i64(stop), w_row = bcast_i64(row);
        const float4 q0 = make_float4(bcast_f(p0.x), bcast_f(p0.y), bcast_f(p0.z), bcast_f(p0.w));
        const float4 q1 = make_float4(bcast_f(p1.x), bcast_f(p1.y), bcast_f(p1.z), bcast_f(p1.w));
        const float4 con = make_float4(bcast_f(conic.x), bcast_f(conic.y), bcast_f(conic.z), bcast_f(conic.w));
        const float2 ctr = make_float2(bcast_f(center.x), bcast_f(center.y));
        const int rad = __builtin_amdgcn_readlane(radius, src);
        const Ellipse we = ellipse_of(q0, q1, ctr, con, rad);
        const int4 bb = we.bounds;
        const bool is_y = (bb.w - bb.y) < (bb.z - bb.x);
        const int s0 = is_y ? bb.y : bb.x, s1 = is_y ? bb.w : bb.z;
        const int full0 = is_y ? bb.x : bb.y, full1 = is_y ? bb.z : bb.w;
        const int view = (int)(w_row / n);
        const uint64_t id = (uint64_t)(uint32_t)(w_row - (int64_t)view * n);
        const uint32_t gbase = (uint32_t)(view * d.gpv);
        const int G0 = s0 >> kGroupShift, G1 = (s1 - 1) >> kGroupShift;
        int64_t base = w_start;
        for (int Gb = G0; Gb <= G1; Gb += 64) {
            const int G = Gb + lane;
            int2 span[1 << kGroupShift];
            int gmin = INT_MAX, gmax = -1;
#pragma unroll
            for (int j = 0; j < (1 << kGroupShift); ++j) {
                span[j] = make_int2(0, 0);
                const int strip = (G << kGroupShift) + j;
                if (G <= G1 && strip >= s0 && strip < s1) {
                    int2 sp = make_int2(full0, full1);
                    if (we.precise)
                        sp = strip_span(we, strip, is_y, line_intersection(we, strip, is_y),
                                        line_intersection(we, strip + 1, is_y));
                    span[j] = sp;
                    if (sp.y > sp.x) {
                        gmin = min(gmin, sp.x >> kGroupShift);
                        gmax = max(gmax, (sp.y - 1) >> kGroupShift);
                    }
                }
            }
            const int cnt = gmax >= gmin ? gmax - gmin + 1 : 0;
            const int incl = wave_inclusive_scan(cnt);
            int64_t p = base + (incl - cnt);
            for (int gc = gmin; gc <= gmax; ++gc) {
                const uint64_t m = group_mask(span, gc, is_y);
                const int GX = is_y ? gc : G, GY = is_y ? G : gc;
                if (p < w_stop) {
                    st_stream(items + p, (id << 32) | (uint64_t)(gbase + (uint32_t)(GY * d.sgx + GX)));
                    st_stream(masks + p, m);
                }
                ++p;
            }
            base += __builtin_amdgcn_readlane(incl, 63);
        }
    }
}

// chunk_base[g] = exclusive scan over groups of ceil(len_g / kChunk);
// chunk_base[groups] = number of chunks.
__global__ __launch_bounds__(1024) void chunk_base_kernel(const int32_t* __restrict__ granges, int groups,
                                                          int32_t* __restrict__ chunk_base) {
    __shared__ int32_t s_wave[1024 / 64];
    int32_t carry = 0;
    for (int base = 0; base < groups; base += 1024) {
        const int g = base + threadIdx.x;
        const int32_t q = g < groups ? (granges[2 * g + 1] - granges[2 * g] + kChunk - 1) / kChunk : 0;
        int32_t total;
        const int32_t ex = block_exclusive_scan<1024>(q, s_wave, total);
        if (g < groups) chunk_base[g] = carry + ex;
        carry += total;
    }
    if (threadIdx.x == 0) chunk_base[groups] = carry;
}

// chunk_group[u] = the group g with chunk_base[g] <= u < chunk_base[g + 1].
__global__ void chunk_group_kernel(const int32_t* __restrict__ chunk_base, int groups, int64_t max_chunks,
                                   int32_t* __restrict__ chunk_group) {
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= max_chunks || u >= chunk_base[groups]) return;
    int lo = 0, hi = groups - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (chunk_base[mid] <= u)
            lo = mid;
        else
            hi = mid - 1;
    }
    chunk_group[u] = lo;
}


// One wavefront per chunk of kChunk items (kChunkSteps per lane, masks and
// ids held in registers).  Counts of group g are laid out [g][tile][chunk]
// starting at 64*chunk_base[g], so one exclusive scan over the whole array
// yields every (tile, chunk) offset within the tile's list.  The wavefront
// walks the tiles its items touch and, per tile, its items in order: one
// ballot per 64 items ranks them, so a tile's run of the chunk is written by
// consecutive stores of one wavefront.
// MASKS: each item's tiles come from masks[] (AccuTile), else from the
// clipped rectangle packed in the item.
// WRITE = false: counts[(g, t, s)] = items of chunk s touching tile t.
// WRITE = true: every item's Gaussian index goes to
//   tile_start[t] + (scanned[(g,t,s)] - scanned[(g,t,0)]) + rank.
// BUF (WRITE, id lists under 4 GiB): a tile's run of the chunk is gathered
// in the wavefront's LDS slice (one ballot-ranked write per 64 items) and
// then stored with consecutive lanes (about one full-width store per tile
// instead of one partial store per 64 items); buffer stores take the run's
// start as the scalar offset, and the buffer's range check stands in for the
// id_limit test.  Tiles are walked in two halves so that each membership
// test reads one 32-bit word of the item's mask.
//
// LISTS (write pass): 0 whole lists; 1 each tile's first list_cap(caps[t])
// entries; 2 a redo pass, the whole lists of the tiles flagged in redo
// (redo_count of them); 3 no pass, only the number of group items mode 1
// would load, added to *loaded.
template <bool WRITE, bool MASKS, bool BUF = false, int LISTS = 0>
__global__ __launch_bounds__(kBinThreads) void group_pass_kernel(
    const uint64_t* __restrict__ items, const uint64_t* __restrict__ masks, const int32_t* __restrict__ granges,
    const int32_t* __restrict__ chunk_base,
    const int32_t* __restrict__ chunk_group, int groups, int64_t max_chunks, GridDims d,
    uint32_t* __restrict__ counts, const int32_t* __restrict__ scanned, const int32_t* __restrict__ tile_start,
    int32_t* __restrict__ ids, int64_t id_limit, const int32_t* __restrict__ caps, const int32_t* __restrict__ redo,
    const int32_t* __restrict__ redo_count, const int32_t* __restrict__ totals,
    unsigned long long* __restrict__ loaded, int32_t* __restrict__ clear_count) {
    // A capped pass clears the overflow count of the blend that follows.
    if constexpr (LISTS == 1)
        if (clear_count && blockIdx.x == 0 && threadIdx.x == 0) *clear_count = 0;
    static_assert(LISTS == 0 || WRITE, "caps and redo flags are write-pass arguments");
    // A chunk's run for one tile, then one slot per lane that rejected items
    // are written to (so the writes need neither a branch nor an exec mask).
    __shared__ int32_t s_run[WRITE && BUF ? kBinWaves : 1][WRITE && BUF ? kChunk + 64 : 1];
    // Counting rectangles: a 9x9 difference grid per wavefront.
    constexpr bool RECT_COUNT = !WRITE && !MASKS;
    __shared__ int32_t s_diff[RECT_COUNT ? kBinWaves : 1][RECT_COUNT ? 96 : 1];
    const int lane = lane_id();
    // One chunk of items per wavefront.  A redo pass (LISTS 2) walks the
    // chunks over a small grid and leaves at once when no tile is flagged.
    auto pass = [&](const int64_t u) {
        if (u >= max_chunks) return;
        if (u >= chunk_base[groups]) {
            // Chunks beyond the last group's: their counts (the tail of the
            // scanned table) are zero.
            if constexpr (!WRITE) counts[u * 64 + lane] = 0u;
            return;
        }
        if constexpr (RECT_COUNT) {
            // Counts of a chunk of rectangle items: each item adds its
            // rectangle's four corners to a difference grid; the 2D prefix sum of
            // the grid at tile t is the number of items covering t.
            int32_t* diff = s_diff[threadIdx.x >> 6];
            const int g = chunk_group[u];
            const int32_t cb = chunk_base[g];
            const int32_t q = chunk_base[g + 1] - cb;
            const int32_t s = (int32_t)(u - cb);
            const int64_t begin = (int64_t)granges[2 * g] + (int64_t)s * kChunk;
            const int64_t end = min(begin + kChunk, (int64_t)granges[2 * g + 1]);
            for (int e = lane; e < 96; e += 64) diff[e] = 0;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // All loads first, from clamped addresses (begin < end): a guarded
            // load would be a branch that waits for its data.
            uint64_t got[kChunkSteps];
#pragma unroll
            for (int k = 0; k < kChunkSteps; ++k) got[k] = items[min(begin + k * 64 + lane, end - 1)];
            // Corners in row or column 8 lie outside the summed 8x8 part and are
            // not added; items starting at the group's first tile (common: the
            // rectangles clipped by the group's edges) add their corner with one
            // atomic per step instead of as many serialised ones on one word.
#pragma unroll
            for (int k = 0; k < kChunkSteps; ++k) {
                const bool in = begin + k * 64 + lane < end;
                const uint32_t local = (uint32_t)(got[k] >> kGroupBits) & 0xFFFu;
                const int lx0 = local & 7, lx1 = ((local >> 3) & 7) + 1, ly0 = (local >> 6) & 7,
                          ly1 = ((local >> 9) & 7) + 1;
                const uint64_t origin = __ballot(in && (lx0 | ly0) == 0);
                if (origin && lane == (int)__builtin_ctzll(origin)) atomicAdd(&diff[0], (int)__popcll(origin));
                if (in) {
                    if ((lx0 | ly0) != 0) atomicAdd(&diff[ly0 * 9 + lx0], 1);
                    if (lx1 < 8) atomicAdd(&diff[ly0 * 9 + lx1], -1);
                    if (ly1 < 8) atomicAdd(&diff[ly1 * 9 + lx0], -1);
                    if (lx1 < 8 && ly1 < 8) atomicAdd(&diff[ly1 * 9 + lx1], 1);
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // Inclusive 2D prefix sum of the grid's 8x8 corner: along each row of
            // 8 lanes, then down the columns (lanes 8 apart).
            const int tx = lane & 7;
            int32_t c = diff[(lane >> 3) * 9 + tx];
#pragma unroll
            for (int d = 1; d < 8; d <<= 1) {
                const int32_t u = __shfl_up(c, d, 8);
                if (tx >= d) c += u;
            }
#pragma unroll
            for (int d = 8; d < 64; d <<= 1) {
                const int32_t u = __shfl_up(c, d, 64);
                if (lane >= d) c += u;
            }
            counts[(int64_t)cb * 64 + (int64_t)lane * q + s] = (uint32_t)c;
            return;
        }
        int32_t* const run_lds = s_run[WRITE && BUF ? threadIdx.x >> 6 : 0];
        const int g = chunk_group[u];
        const int32_t cb = chunk_base[g];
        const int32_t q = chunk_base[g + 1] - cb;
        const int32_t s = (int32_t)(u - cb);
        const int64_t begin = (int64_t)granges[2 * g] + (int64_t)s * kChunk;
        const int64_t end = min(begin + kChunk, (int64_t)granges[2 * g + 1]);
        const int64_t slot = (int64_t)cb * 64 + (int64_t)lane * q;  // entry (g, lane, 0)
        // Write pass: lane t's tile starts this chunk's run at init and keeps its
        // first `limit` ids.  With caps, a tile keeps the first list_cap(caps[t])
        // entries of its list; a redo pass writes only the flagged tiles, in
        // full.  Chunks that no tile needs return before loading their items.
        uint32_t init = 0, limit = 0xFFFFFFFFu;
        uint64_t want_tiles = ~0ull;
        if constexpr (WRITE) {
            const int view = g / d.gpv, rem = g - view * d.gpv;
            const int Y = rem / d.sgx, X = rem - Y * d.sgx;
            const int ty = (Y << kGroupShift) + (lane >> 3), tx = (X << kGroupShift) + (lane & 7);
            const bool inside = ty < d.gy && tx < d.gx;
            const int64_t gt = (int64_t)view * d.tpv + ty * d.gx + tx;
            // A redo pass reads its flags before anything else: most chunks have
            // no flagged tile.
            bool want = inside && (LISTS != 2 || redo[gt] != 0);
            if (LISTS == 2 && __ballot(want) == 0) return;
            if (inside) {
                const uint32_t rel = (uint32_t)(scanned[slot + s] - scanned[slot]);
                init = (uint32_t)tile_start[gt] + rel;
                if constexpr (LISTS == 1 || LISTS == 3) {
                    // Wanted while the tile has entries left below its cap
                    // (a tile whose list ends first stops wanting chunks).
                    const uint32_t cap = list_cap(caps[gt]);
                    want = rel < min(cap, (uint32_t)totals[gt]);
                    limit = want ? cap - rel : 0u;
                }
            }
            if constexpr (LISTS != 0) {
                want_tiles = __ballot(want);
                if constexpr (LISTS == 3) {
                    if (lane == 0 && want_tiles) atomicAdd(loaded, (unsigned long long)(end - begin));
                    return;
                }
                if (want_tiles == 0) return;
            }
        }
        uint64_t mask[kChunkSteps];
        int32_t id[kChunkSteps];
        uint64_t any = 0;
        // All loads first, from clamped addresses (begin < end), then the lanes
        // beyond the chunk's end are cleared.
        uint64_t got[kChunkSteps];
#pragma unroll
        for (int k = 0; k < kChunkSteps; ++k) {
            const int64_t i = min(begin + k * 64 + lane, end - 1);
            got[k] = items[i];
            if constexpr (MASKS) mask[k] = masks[i];
        }
#pragma unroll
        for (int k = 0; k < kChunkSteps; ++k) {
            const bool in = begin + k * 64 + lane < end;
            if constexpr (!MASKS) mask[k] = group_tile_mask((uint32_t)(got[k] >> kGroupBits) & 0xFFFu);
            if (!in) mask[k] = 0;
            id[k] = in ? (int32_t)(got[k] >> 32) : 0;
            any |= mask[k];
        }
        uint32_t mine = 0;
        const uint64_t todo_all = LISTS != 0 ? wave_or64(any) & want_tiles : wave_or64(any);
        // (unused unless WRITE && BUF)
        const __amdgpu_buffer_rsrc_t rsrc =
            __builtin_amdgcn_make_buffer_rsrc(ids, (short)0, (int)(uint32_t)(BUF ? id_limit * 4 : 0), 0x00020000);
        auto walk = [&](auto half) {
            constexpr int H = decltype(half)::value;
            uint32_t todo = (uint32_t)(todo_all >> (32 * H));
            while (todo) {
                const int tb = __builtin_ctz(todo);
                todo &= todo - 1;
                const int t = 32 * H + tb;
                const uint32_t bit = 1u << tb;
                const uint32_t start = WRITE ? (uint32_t)__builtin_amdgcn_readlane((int)init, t) : 0u;
                const uint32_t lim = LISTS == 1 ? (uint32_t)__builtin_amdgcn_readlane((int)limit, t) : 0xFFFFFFFFu;
                uint32_t run = WRITE && BUF ? 0u : start;
#pragma unroll
                for (int k = 0; k < kChunkSteps; ++k) {
                    const uint32_t word = H ? (uint32_t)(mask[k] >> 32) : (uint32_t)mask[k];
                    const bool has = (word & bit) != 0u;
                    const uint64_t b = __ballot(has);
                    if constexpr (WRITE && BUF) {
                        const uint32_t rank =
                            __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
                        run_lds[has ? run + rank : (uint32_t)(kChunk + lane)] = id[k];
                        run += (uint32_t)__popcll(b);
                    } else if (b) {
                        if constexpr (WRITE) {
                            if (has) {
                                const uint32_t rank = __builtin_amdgcn_mbcnt_hi(
                                    (uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
                                const int64_t pos = (int64_t)run + rank;
                                if (pos < id_limit && (uint32_t)(pos - start) < lim)
                                    ids[pos] = id[k];  // plain: short runs per tile, merged in L2
                            }
                        }
                        run += (uint32_t)__popcll(b);
                    }
                }
                if constexpr (WRITE && BUF) {
                    // The run is complete in LDS: store it with consecutive lanes.
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    const uint32_t keep = min(run, lim);
                    for (uint32_t e = (uint32_t)lane; e < keep; e += 64)
                        __builtin_amdgcn_raw_buffer_store_b32(run_lds[e], rsrc, (int)(e * 4u), (int)(start * 4u), 0);
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                }
                if (lane == t) mine = run;
            }
        };
        // Buffered write: the tiles of each half are visited from the highest bit
        // down and every step's mask word is shifted left as the walk proceeds, so
        // one add of the word to itself both advances it and yields the tile's
        // membership bit as its carry (the carry mask is the ballot).  Each step
        // then costs the carry add, the two-part lane count, one address and one
        // select; non-members write to their own slot beyond the run.
        auto walk_buf = [&](auto half) {
            constexpr int H = decltype(half)::value;
            static_assert(kChunk % 128 == 0, "store loop reads two 64-word rows below kChunk");
            uint32_t todo = (uint32_t)(todo_all >> (32 * H));
            uint32_t w[kChunkSteps];
#pragma unroll
            for (int k = 0; k < kChunkSteps; ++k) w[k] = (uint32_t)(mask[k] >> (32 * H));
            using lds_i32 = __attribute__((address_space(3))) int32_t;
            // LDS byte addresses: the slice's first word (wave-uniform) and this
            // lane's spare slot.
            const uint32_t slice_word =
                (uint32_t)__builtin_amdgcn_readfirstlane((int)((uint32_t)(uintptr_t)(lds_i32*)run_lds >> 2));
            const uint32_t spare = (slice_word + (uint32_t)(kChunk + lane)) << 2;
            int top = 31;  // bit of the original word now at bit 31 of w[]
            while (todo) {
                const int tb = 31 - __builtin_clz(todo);
                todo ^= 1u << tb;
                const int sh = top - tb;
                if (sh != 0) {
#pragma unroll
                    for (int k = 0; k < kChunkSteps; ++k) w[k] <<= sh;
                }
                top = tb - 1;
                const int t = 32 * H + tb;
                const uint32_t start = (uint32_t)__builtin_amdgcn_readlane((int)init, t);
                const uint32_t lim = LISTS == 1 ? (uint32_t)__builtin_amdgcn_readlane((int)limit, t) : 0xFFFFFFFFu;
                uint32_t end_word = slice_word;  // LDS word after the run so far
#pragma unroll
                for (int k = 0; k < kChunkSteps; ++k) {
                    // b = carry mask of w + w: lanes whose item covers tile t.
                    uint32_t next;
                    uint64_t b;
                    asm volatile("v_add_co_u32_e64 %0, %1, %2, %2" : "=v"(next), "=s"(b) : "v"(w[k]));
                    w[k] = next;
                    const uint32_t rank =
                        __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
                    const uint32_t member = (rank + end_word) << 2;
                    uint32_t at;
                    asm volatile("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(at) : "v"(spare), "v"(member), "s"(b));
                    *(lds_i32*)(uintptr_t)at = id[k];
                    end_word += (uint32_t)__popcll(b);
                }
                const uint32_t run = min(end_word - slice_word, lim);  // ids this chunk keeps for tile t
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                // Two LDS reads in flight per lane before the stores: a run holds
                // at most kChunk ids, so e0 <= kChunk - 128 and both reads stay in
                // the slice (words past the run are read but not stored).
                for (uint32_t e0 = 0; e0 < run; e0 += 128) {
                    const uint32_t e1 = e0 + (uint32_t)lane, e2 = e1 + 64u;
                    int32_t v1 = run_lds[e1], v2 = run_lds[e2];
                    asm volatile("" : "+v"(v1), "+v"(v2));  // both reads issued before either store
                    if (e1 < run) __builtin_amdgcn_raw_buffer_store_b32(v1, rsrc, (int)(e1 * 4u), (int)(start * 4u), 0);
                    if (e2 < run) __builtin_amdgcn_raw_buffer_store_b32(v2, rsrc, (int)(e2 * 4u), (int)(start * 4u), 0);
                }
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                __builtin_amdgcn_wave_barrier();
            }
        };
        if constexpr (WRITE && BUF) {
            walk_buf(std::integral_constant<int, 0>{});
            walk_buf(std::integral_constant<int, 1>{});
        } else {
            walk(std::integral_constant<int, 0>{});
            walk(std::integral_constant<int, 1>{});
        }
        if constexpr (!WRITE) counts[slot + s] = mine;
    };
    if constexpr (LISTS == 2) {
        if (*redo_count == 0) return;
        const int64_t waves = (int64_t)gridDim.x * kBinWaves;
        for (int64_t u = (int64_t)blockIdx.x * kBinWaves + (threadIdx.x >> 6); u < max_chunks; u += waves) pass(u);
    } else {
        pass(xcd_contiguous(blockIdx.x, gridDim.x) * kBinWaves + (threadIdx.x >> 6));
    }
}

// Pairs of global tile `tile`: the sum over its group's chunks.
GS3D_DEV int32_t tile_total(const int32_t* __restrict__ chunk_base, const uint32_t* __restrict__ counts,
                            const int32_t* __restrict__ scanned, const GridDims& d, int64_t tile) {
    const int view = (int)(tile / d.tpv);
    const int r = (int)(tile - (int64_t)view * d.tpv);
    const int ty = r / d.gx, tx = r - ty * d.gx;
    const int g = view * d.gpv + (ty >> kGroupShift) * d.sgx + (tx >> kGroupShift);
    const int t = ((ty & 7) << 3) + (tx & 7);
    const int32_t cb = chunk_base[g];
    const int32_t q = chunk_base[g + 1] - cb;
    if (q <= 0) return 0;
    const int64_t first = (int64_t)cb * 64 + (int64_t)t * q;
    const int64_t last = first + q - 1;
    return scanned[last] + (int32_t)counts[last] - scanned[first];
}

__global__ void tile_totals_kernel(const int32_t* __restrict__ chunk_base, const uint32_t* __restrict__ counts,
                                   const int32_t* __restrict__ scanned, GridDims d, int64_t tiles,
                                   int32_t* __restrict__ totals) {
    const int64_t tile = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (tile >= tiles) return;
    totals[tile] = tile_total(chunk_base, counts, scanned, d, tile);
}

__global__ void tile_ranges_from_totals_kernel(const int32_t* __restrict__ totals, const int32_t* __restrict__ starts,
                                               int64_t tiles, int32_t* __restrict__ ranges) {
    const int64_t tile = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (tile >= tiles) return;
    const int32_t n = totals[tile];
    const int32_t a = n > 0 ? starts[tile] : 0;
    reinterpret_cast<int2*>(ranges)[tile] = make_int2(a, a + n);
}

// tiles[p] = t for every p in [ranges[t][0], ranges[t][1]); one block per tile.
__global__ void pair_tiles_kernel(const int32_t* __restrict__ ranges, int64_t tile_count, uint32_t* __restrict__ out,
                                  int64_t count) {
    const int64_t tile = blockIdx.x;
    const int32_t a = ranges[2 * tile], b = ranges[2 * tile + 1];
    for (int64_t p = (int64_t)a + threadIdx.x; p < b; p += blockDim.x)
        if (p < count) out[p] = (uint32_t)tile;
}

// 64-bit reference keys (tile << 32 | depth bits) of sorted (tile, id) pairs.
__global__ void expand_keys_kernel(const uint32_t* __restrict__ tiles, const int32_t* __restrict__ ids,
                                   int64_t count, const float* __restrict__ depths, int n, int tiles_per_view,
                                   uint64_t* __restrict__ keys) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const uint32_t tile = tiles[i];
    const int64_t view = tile / (uint32_t)tiles_per_view;
    keys[i] = ((uint64_t)tile << 32) | (uint64_t)__float_as_uint(depths[view * n + ids[i]]);
}

// Scratch of gs3d_order_rows.
struct OrderScratch {
    uint32_t* keys;       // 2*rows depth-bit keys
    int32_t* counts;      // rows group counts
    int64_t* pairs;       // per-block tile pair counts
    int64_t* live;        // rows that the depth order keeps (outside AccuTile)
    uint32_t* range;      // per sort tile: smallest and largest kept key
    uint32_t* base;       // key base of the passes after the first (key_base_kernel)
    void* sort;
    void* scan;
};

inline size_t order_scratch_bytes(int64_t rows, OrderScratch* out, void* base) {
    const int64_t blocks = (rows + kBinThreads - 1) / kBinThreads;
    const int64_t sort_tiles = (rows + kSortTile - 1) / kSortTile;
    const size_t a = align256((size_t)rows * 2 * sizeof(uint32_t));
    const size_t b = align256((size_t)rows * sizeof(int32_t));
    const size_t c = align256((size_t)blocks * sizeof(int64_t));
    const size_t l = align256(sizeof(int64_t));
    const size_t r = align256((size_t)sort_tiles * 2 * sizeof(uint32_t));
    const size_t e = align256(sort_scratch_bytes(rows, nullptr, nullptr, kOrderRadixBits));
    const size_t f = scan_partials_bytes(rows);
    if (out) {
        char* p = reinterpret_cast<char*>(base);
        out->keys = reinterpret_cast<uint32_t*>(p);
        out->counts = reinterpret_cast<int32_t*>(p + a);
        out->pairs = reinterpret_cast<int64_t*>(p + a + b);
        out->live = reinterpret_cast<int64_t*>(p + a + b + c);
        out->range = reinterpret_cast<uint32_t*>(p + a + b + c + l);
        out->base = reinterpret_cast<uint32_t*>(p + a + b + c + l + r);
        out->sort = p + a + b + c + l + r + l;
        out->scan = p + a + b + c + l + r + l + e;
    }
    return a + b + c + l + r + l + e + f;
}

// Scratch of gs3d_bin_rows.
struct BinScratch {
    uint64_t* masks;      // 2*group_pairs tile masks (AccuTile only)
    uint64_t* items;      // 2*group_pairs
    void* sort;
    int32_t* granges;     // 2*groups
    int32_t* chunk_base;  // groups + 1
    int32_t* chunk_group; // max_chunks
    uint32_t* counts;     // 64*max_chunks
    int32_t* scanned;     // 64*max_chunks
    int32_t* totals;      // tiles
    int32_t* starts;      // tiles
    void* scan;
};

inline int64_t max_chunks_of(int64_t group_pairs, int64_t groups) { return (group_pairs + kChunk - 1) / kChunk + groups; }

inline size_t bin_scratch_bytes(int64_t group_pairs, int64_t groups, int64_t tiles, bool masks, BinScratch* out,
                                void* base) {
    const int64_t chunks = max_chunks_of(group_pairs, groups);
    size_t sizes[11];
    sizes[0] = align256((size_t)group_pairs * 2 * sizeof(uint64_t));
    sizes[1] = align256(sort_scratch_bytes(group_pairs, nullptr, nullptr,
                                           groups <= (int64_t)1 << kOnePassBits ? kOnePassBits : 8));
    sizes[2] = align256((size_t)groups * 2 * sizeof(int32_t));
    sizes[3] = align256((size_t)(groups + 1) * sizeof(int32_t));
    sizes[4] = align256((size_t)chunks * sizeof(int32_t));
    sizes[5] = align256((size_t)chunks * 64 * sizeof(uint32_t));
    sizes[6] = sizes[5];
    sizes[7] = align256((size_t)tiles * sizeof(int32_t));
    sizes[8] = sizes[7];
    const size_t scan_a = scan_partials_bytes(chunks * 64), scan_b = scan_partials_bytes(tiles);
    sizes[9] = scan_a > scan_b ? scan_a : scan_b;
    sizes[10] = masks ? align256((size_t)group_pairs * 2 * sizeof(uint64_t)) : 0;
    size_t total = 0;
    char* p = reinterpret_cast<char*>(base);
    void* parts[11];
    for (int k = 0; k < 11; ++k) {
        parts[k] = p ? p + total : nullptr;
        total += sizes[k];
    }
    if (out) {
        out->items = reinterpret_cast<uint64_t*>(parts[0]);
        out->sort = parts[1];
        out->granges = reinterpret_cast<int32_t*>(parts[2]);
        out->chunk_base = reinterpret_cast<int32_t*>(parts[3]);
        out->chunk_group = reinterpret_cast<int32_t*>(parts[4]);
        out->counts = reinterpret_cast<uint32_t*>(parts[5]);
        out->scanned = reinterpret_cast<int32_t*>(parts[6]);
        out->totals = reinterpret_cast<int32_t*>(parts[7]);
        out->starts = reinterpret_cast<int32_t*>(parts[8]);
        out->scan = parts[9];
        out->masks = masks ? reinterpret_cast<uint64_t*>(parts[10]) : nullptr;
    }
    return total;
}

// Tile mode and conics of an entry point: conics are required (16-byte
// aligned) outside the radius mode.
inline int check_tile_mode(int mode, const float* conics) {
    if (mode < GS3D_TILE_RADIUS || mode > GS3D_TILE_ACCUTILE) return GS3D_ERR_ARGUMENT;
    if (mode != GS3D_TILE_RADIUS && (!conics || (reinterpret_cast<uintptr_t>(conics) & 15))) return GS3D_ERR_ARGUMENT;
    return GS3D_OK;
}

inline int bit_length(int64_t v) {
    int b = 0;
    while (v > 0) {
        ++b;
        v >>= 1;
    }
    return b;
}

}  // namespace gs3d

extern "C" size_t gs3d_scan_scratch_bytes(int64_t n) { return gs3d::scan_partials_bytes(n < 0 ? 0 : n); }

extern "C" int gs3d_scan_i32(const int32_t* counts, int64_t n, int32_t* offsets, int64_t* total, void* scratch,
                             size_t scratch_bytes, void* stream) {
    if (n < 0) return GS3D_ERR_ARGUMENT;
    if (n == 0) return GS3D_OK;
    if (!counts || !offsets || !scratch) return GS3D_ERR_ARGUMENT;
    if (scratch_bytes < gs3d::scan_partials_bytes(n)) return GS3D_ERR_SCRATCH;
    return gs3d::run_scan<int32_t, true>(counts, n, offsets, total, scratch, gs3d::as_stream(stream));
}

extern "C" size_t gs3d_emit_scratch_bytes(int64_t rows) {
    return gs3d::align256(256 + (size_t)(rows < 0 ? 0 : rows) * 4);
}

extern "C" int gs3d_emit_keys(const gs3d_emit_args* args, void* scratch, size_t scratch_bytes, void* stream) {
    if (!args) return GS3D_ERR_ARGUMENT;
    const gs3d_emit_args& a = *args;
    if (a.n < 0 || a.views < 0 || a.width <= 0 || a.height <= 0) return GS3D_ERR_ARGUMENT;
    if (gs3d::check_tile_mode(a.tile_mode, a.tile_mode == GS3D_TILE_RADIUS ? nullptr : a.conics) != GS3D_OK)
        return GS3D_ERR_ARGUMENT;
    const int64_t rows = (int64_t)a.n * a.views;
    if (rows == 0) return GS3D_OK;
    if (!a.centers || !a.radii || !a.depths || !a.offsets || !a.keys || !a.values || !scratch)
        return GS3D_ERR_ARGUMENT;
    if (reinterpret_cast<uintptr_t>(a.centers) & 7) return GS3D_ERR_ARGUMENT;
    if (scratch_bytes < gs3d_emit_scratch_bytes(rows)) return GS3D_ERR_SCRATCH;
    const int64_t tiles_total = (int64_t)((a.width + 15) / 16) * ((a.height + 15) / 16) * a.views;
    if (tiles_total > 0xFFFFFFFFll) return GS3D_ERR_OVERFLOW;
    hipStream_t s = gs3d::as_stream(stream);
    if (a.tile_mode == GS3D_TILE_ACCUTILE) {
        hipLaunchKernelGGL(gs3d::emit_accutile_kernel, dim3(gs3d::blocks_for(rows, gs3d::kEmitThreads)),
                           dim3(gs3d::kEmitThreads), 0, s, a);
        return gs3d::launch_status("gs3d_emit_keys");
    }
    uint32_t* queue_count = reinterpret_cast<uint32_t*>(scratch);
    int32_t* queue = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(scratch) + 256);
    gs3d::fill_u32(queue_count, 1, 0u, s);
    hipLaunchKernelGGL(gs3d::emit_small_kernel, dim3(gs3d::blocks_for(rows, gs3d::kEmitThreads)),
                       dim3(gs3d::kEmitThreads), 0, s, a, queue_count, queue);
    hipLaunchKernelGGL(gs3d::emit_large_kernel, dim3(2048), dim3(gs3d::kEmitThreads), 0, s, a, queue_count, queue);
    return gs3d::launch_status("gs3d_emit_keys");
}

extern "C" size_t gs3d_sort_scratch_bytes(int64_t count) {
    return gs3d::sort_scratch_bytes(count < 0 ? 0 : count, nullptr, nullptr);
}

template <class K>
static int sort_entry(K* keys, int32_t* values, int64_t count, int32_t end_bit, void* scratch, size_t scratch_bytes,
                      void* stream, int max_bits) {
    if (count < 0 || end_bit < 0 || end_bit > max_bits) return GS3D_ERR_ARGUMENT;
    if (count <= 1 || end_bit == 0) return GS3D_OK;
    if (count > INT32_MAX) return GS3D_ERR_OVERFLOW;
    if (!keys || !values || !scratch) return GS3D_ERR_ARGUMENT;
    if (scratch_bytes < gs3d_sort_scratch_bytes(count)) return GS3D_ERR_SCRATCH;
    return gs3d::run_sort<K>(keys, values, count, end_bit, scratch, gs3d::as_stream(stream));
}

extern "C" int gs3d_sort_pairs_u64(uint64_t* keys, int32_t* values, int64_t count, int32_t end_bit, void* scratch,
                                   size_t scratch_bytes, void* stream) {
    return sort_entry<uint64_t>(keys, values, count, end_bit, scratch, scratch_bytes, stream, 64);
}

extern "C" int gs3d_sort_pairs_u32(uint32_t* keys, int32_t* values, int64_t count, int32_t end_bit, void* scratch,
                                   size_t scratch_bytes, void* stream) {
    return sort_entry<uint32_t>(keys, values, count, end_bit, scratch, scratch_bytes, stream, 32);
}

// ---------------------------------------------------------------------------
// Allocation-free pair sort (gs3d_sort_pairs_u64_static): the scratch of the
// radix sort lives in this file-scope device array, one copy per GPU, held
// until the process ends.  Host code never passes the array's name to a
// kernel (on the host it is only a stand-in for the symbol): the first call
// on each device, with that device current, resolves the array's device
// address with hipGetSymbolAddress and keeps it per device; every launch
// takes that address.  The sort writes every histogram and scan entry it
// reads, so nothing has to start at zero.  Calls that overlap on one GPU
// (other streams or threads) share the array and race.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char static_scratch[GS3D_STATIC_SCRATCH_BYTES];

namespace gs3d {
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_static_scratch_mutex;
void* g_static_scratch_ptr[kMaxDevices] = {};
}  // namespace

// Device address of static_scratch on the device of `stream` (which must be
// the current device).
static int static_scratch_address(hipStream_t stream, void** out) {
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) {
        set_error("gs3d_sort_pairs_u64_static: no usable current device");
        return GS3D_ERR_LAUNCH;
    }
    if (stream) {
        hipDevice_t stream_device = -1;
        if (hipStreamGetDevice(stream, &stream_device) != hipSuccess || stream_device != device) {
            set_error("gs3d_sort_pairs_u64_static: the stream must belong to the current device");
            return GS3D_ERR_ARGUMENT;
        }
    }
    std::lock_guard<std::mutex> lock(g_static_scratch_mutex);
    if (!g_static_scratch_ptr[device]) {
        void* address = nullptr;
        const hipError_t err = hipGetSymbolAddress(&address, HIP_SYMBOL(static_scratch));
        if (err != hipSuccess || !address) {
            set_error("gs3d_sort_pairs_u64_static: hipGetSymbolAddress of the static scratch failed");
            return GS3D_ERR_LAUNCH;
        }
        g_static_scratch_ptr[device] = address;
    }
    *out = g_static_scratch_ptr[device];
    return GS3D_OK;
}
}  // namespace gs3d

extern "C" int gs3d_sort_pairs_u64_static(uint64_t* keys, int32_t* values, int64_t count, int32_t end_bit,
                                          void* stream) {
    if (count < 0 || end_bit < 0 || end_bit > 64) return GS3D_ERR_ARGUMENT;
    if (count <= 1 || end_bit == 0) return GS3D_OK;
    if (count > INT32_MAX) return GS3D_ERR_OVERFLOW;
    if (!keys || !values) return GS3D_ERR_ARGUMENT;
    if (gs3d_sort_scratch_bytes(count) > (size_t)GS3D_STATIC_SCRATCH_BYTES) {
        gs3d::set_error("gs3d_sort_pairs_u64_static: count needs more scratch than GS3D_STATIC_SCRATCH_BYTES");
        return GS3D_ERR_SCRATCH;
    }
    void* scratch = nullptr;
    hipStream_t s = gs3d::as_stream(stream);
    const int status = gs3d::static_scratch_address(s, &scratch);
    if (status != GS3D_OK) return status;
    return gs3d::run_sort<uint64_t>(keys, values, count, end_bit, scratch, s);
}

extern "C" int gs3d_tile_ranges(const uint64_t* sorted_keys, int64_t count, int32_t* ranges, int64_t tile_count,
                                void* stream) {
    if (count < 0 || tile_count < 0) return GS3D_ERR_ARGUMENT;
    if (count == 0) return GS3D_OK;
    if (!sorted_keys || !ranges) return GS3D_ERR_ARGUMENT;
    hipLaunchKernelGGL(gs3d::tile_ranges_kernel<uint64_t>, dim3(gs3d::blocks_for(count, 256)), dim3(256), 0,
                       gs3d::as_stream(stream), sorted_keys, count, 32, 0xFFFFFFFFu, ranges, tile_count);
    return gs3d::launch_status("gs3d_tile_ranges");
}

extern "C" size_t gs3d_order_rows_scratch_bytes(int64_t rows) {
    return gs3d::order_scratch_bytes(rows < 0 ? 0 : rows, nullptr, nullptr);
}

extern "C" int gs3d_order_rows(const gs3d_order_args* args, void* scratch, size_t scratch_bytes, void* stream) {
    if (!args) return GS3D_ERR_ARGUMENT;
    const gs3d_order_args& a = *args;
    if (a.n < 0 || a.views < 0 || a.width <= 0 || a.height <= 0 || !a.totals) return GS3D_ERR_ARGUMENT;
    const int64_t rows = (int64_t)a.n * a.views;
    hipStream_t s = gs3d::as_stream(stream);
    if (a.sort_bits < 0 || a.sort_bits > 32) return GS3D_ERR_ARGUMENT;
    if (rows == 0) {
        gs3d::fill_u32(reinterpret_cast<uint32_t*>(a.totals), 4, 0u, s);
        if (a.key_bits_out) gs3d::fill_u32(reinterpret_cast<uint32_t*>(a.key_bits_out), 1, 0u, s);
        return gs3d::launch_status("gs3d_order_rows");
    }
    if (rows > INT32_MAX) return GS3D_ERR_OVERFLOW;
    const gs3d::GridDims d = gs3d::grid_dims(a.width, a.height);
    if (d.gx >= 0xFFFF || d.gy >= 0xFFFF) return GS3D_ERR_UNSUPPORTED;
    if (!a.depths || !a.centers || !a.radii || !a.order || !a.group_offsets || !scratch) return GS3D_ERR_ARGUMENT;
    if ((reinterpret_cast<uintptr_t>(a.centers) & 7) || (reinterpret_cast<uintptr_t>(a.order) & 7))
        return GS3D_ERR_ARGUMENT;
    if (gs3d::check_tile_mode(a.tile_mode, a.conics) != GS3D_OK) return GS3D_ERR_ARGUMENT;
    if (scratch_bytes < gs3d_order_rows_scratch_bytes(rows)) return GS3D_ERR_SCRATCH;
    gs3d::OrderScratch sc;
    gs3d::order_scratch_bytes(rows, &sc, scratch);
    const gs3d::RowGeometry geo{a.centers, a.conics, a.radii, a.tile_mode};
    const bool accu = a.tile_mode == GS3D_TILE_ACCUTILE;
    const bool packed = d.gx <= 256 && d.gy <= 256;
    // Key bits the depth order sorts (at least 9: its first two passes).
    const int end_bit = a.sort_bits == 0 ? 32 : (a.sort_bits < 9 ? 9 : a.sort_bits);
    int shifts[4], widths[4];
    // The records are written to the half that leaves the sorted result in
    // the first half of keys and order after the passes.
    const int start_half = accu ? 0 : gs3d::order_passes(end_bit, shifts, widths) & 1;
    if (accu && (!a.footprints || (reinterpret_cast<uintptr_t>(a.footprints) & 15))) return GS3D_ERR_ARGUMENT;
    float4* fp = reinterpret_cast<float4*>(a.footprints);
    const dim3 grid(gs3d::blocks_for(rows, 256)), block(256);
    if (accu && packed)
        hipLaunchKernelGGL((gs3d::row_records_kernel<true>), grid, block, 0, s, a.depths, geo, rows, d.gx, d.gy,
                           sc.keys, a.order, a.tiles_out, fp);
    else if (accu)
        hipLaunchKernelGGL((gs3d::row_records_kernel<false>), grid, block, 0, s, a.depths, geo, rows, d.gx, d.gy,
                           sc.keys, a.order, a.tiles_out, fp);
    else {
        // Outside AccuTile the records kernel also forms the depth order's
        // first digit counts.
        gs3d::SortScratch ss;
        gs3d::sort_scratch_bytes(rows, &ss, sc.sort, gs3d::kOrderRadixBits);
        const int64_t tiles = (rows + gs3d::kSortTile - 1) / gs3d::kSortTile;
        uint32_t* keys_in = sc.keys + start_half * rows;
        uint64_t* records_in = a.order + start_half * rows;
        if (packed)
            hipLaunchKernelGGL((gs3d::row_records_counted_kernel<true>), dim3((unsigned)tiles),
                               dim3(gs3d::kSortThreads), 0, s, a.depths, geo, rows, d.gx, d.gy, keys_in, records_in,
                               a.tiles_out, ss.counts, tiles, sc.range);
        else
            hipLaunchKernelGGL((gs3d::row_records_counted_kernel<false>), dim3((unsigned)tiles),
                               dim3(gs3d::kSortThreads), 0, s, a.depths, geo, rows, d.gx, d.gy, keys_in, records_in,
                               a.tiles_out, ss.counts, tiles, sc.range);
        hipLaunchKernelGGL(gs3d::key_base_kernel, dim3(1), dim3(1024), 0, s, sc.range, tiles, sc.base,
                           a.key_bits_out);
    }
    if (accu && a.key_bits_out)
        hipLaunchKernelGGL(gs3d::key_base_kernel, dim3(1), dim3(1024), 0, s, (const uint32_t*)nullptr, (int64_t)0,
                           sc.base, a.key_bits_out);
    // order holds 2*rows records: [0, rows) sorted result, [rows, 2rows) ping-pong.  With packed
    // records the last pass also writes each row's group count at its sorted position and the
    // blocks' tile-pair sums; otherwise order_counts_kernel computes them from the geometry.
    // Outside AccuTile the rows that touch no tile are left out of the sort; their places at
    // the end hold filler records (row 0, no rectangle) with no groups.
    const int tail_kind = packed ? (accu ? 2 : 1) : 0;
    // The last pass writes 16-bit group counts (packed records); order_counts_kernel
    // writes 32-bit ones.
    uint16_t* const counts16 = reinterpret_cast<uint16_t*>(sc.counts);
    int status;
    if (accu)
        status = gs3d::run_sort<uint32_t, uint64_t>(sc.keys, a.order, rows, 32, sc.sort, s, tail_kind,
                                                    gs3d::OrderTail{counts16, sc.pairs});
    else
        status = gs3d::run_order_sort(sc.keys, a.order, rows, sc.sort, sc.live,
                                      packed ? (uint64_t)gs3d::kEmptyRect << 32 : 0u, s, tail_kind,
                                      gs3d::OrderTail{counts16, sc.pairs}, true, end_bit, start_half, sc.base);
    if (status != GS3D_OK) return status;
    int64_t pair_blocks = (rows + gs3d::kSortTile - 1) / gs3d::kSortTile;
    if (!packed) {
        const dim3 cgrid(gs3d::blocks_for(rows, gs3d::kBinThreads)), cblock(gs3d::kBinThreads);
        if (accu)
            hipLaunchKernelGGL((gs3d::order_counts_kernel<false, true>), cgrid, cblock, 0, s, a.order, rows, geo, d.gx,
                               d.gy, sc.counts, sc.pairs, (const int64_t*)nullptr);
        else
            hipLaunchKernelGGL((gs3d::order_counts_kernel<false, false>), cgrid, cblock, 0, s, a.order, rows, geo,
                               d.gx, d.gy, sc.counts, sc.pairs, (const int64_t*)sc.live);
        pair_blocks = cgrid.x;
    }
    // The blocks' tile-pair sums are added up by the group-count scan's first launch.
    const gs3d::SideSum pair_sum{sc.pairs, pair_blocks, a.totals + 1};
    status = packed ? gs3d::run_scan<uint16_t, true>(counts16, rows, a.group_offsets, a.totals, sc.scan, s, pair_sum)
                    : gs3d::run_scan<int32_t, true>(sc.counts, rows, a.group_offsets, a.totals, sc.scan, s, pair_sum);
    if (status != GS3D_OK) return status;
    return gs3d::launch_status("gs3d_order_rows");
}

extern "C" size_t gs3d_bin_rows_scratch_bytes(int64_t group_pairs, int32_t views, int32_t width, int32_t height,
                                              int32_t tile_mode) {
    if (group_pairs < 0 || views < 0 || width <= 0 || height <= 0) return 0;
    const gs3d::GridDims d = gs3d::grid_dims(width, height);
    return gs3d::bin_scratch_bytes(group_pairs, (int64_t)views * d.gpv, (int64_t)views * d.tpv,
                                   tile_mode == GS3D_TILE_ACCUTILE, nullptr, nullptr);
}

namespace gs3d {

// Group items of depth-ordered rectangle rows (radius and SnugBox modes):
// at most S of them, written to the start of the binning scratch, where the
// group sort reads them.
inline void emit_group_items(const gs3d_bin_args& a, const GridDims& d, int64_t S, uint64_t* items, hipStream_t s) {
    const int64_t rows = (int64_t)a.n * a.views;
    const RowGeometry geo{a.centers, a.conics, a.radii, a.tile_mode};
    const dim3 egrid(blocks_for(rows, kBinThreads)), eblock(kBinThreads);
    if (d.gx <= 256 && d.gy <= 256)
        hipLaunchKernelGGL(group_emit_kernel<true>, egrid, eblock, 0, s, a.order, a.group_offsets, rows, geo, a.n, d, S,
                           items);
    else
        hipLaunchKernelGGL(group_emit_kernel<false>, egrid, eblock, 0, s, a.order, a.group_offsets, rows, geo, a.n, d,
                           S, items);
}

// gs3d_bin_rows; with `emitted` the group items are already in the scratch
// (gs3d_emit_group_items with a capacity of at least group_pairs).
int write_pass(const gs3d_bin_args& a, const BinScratch& sc, const uint64_t* items, int64_t groups, int64_t chunks,
               const GridDims& d, const int32_t* caps, const int32_t* redo, const int32_t* redo_count, hipStream_t s);

int bin_rows(const gs3d_bin_args* args, void* scratch, size_t scratch_bytes, void* stream, bool emitted) {
    if (!args) return GS3D_ERR_ARGUMENT;
    const gs3d_bin_args& a = *args;
    if (emitted && a.tile_mode == GS3D_TILE_ACCUTILE) return GS3D_ERR_ARGUMENT;
    if (a.n < 0 || a.views < 0 || a.width <= 0 || a.height <= 0 || a.group_pairs < 0 || a.tile_pairs < 0)
        return GS3D_ERR_ARGUMENT;
    if (gs3d::check_tile_mode(a.tile_mode, a.tile_mode == GS3D_TILE_RADIUS ? nullptr : a.conics) != GS3D_OK)
        return GS3D_ERR_ARGUMENT;
    const gs3d::GridDims d = gs3d::grid_dims(a.width, a.height);
    const int64_t rows = (int64_t)a.n * a.views;
    const int64_t groups = (int64_t)a.views * d.gpv, tiles = (int64_t)a.views * d.tpv;
    if (tiles == 0) return GS3D_OK;
    if (!a.ranges) return GS3D_ERR_ARGUMENT;
    if (rows > INT32_MAX || a.group_pairs > INT32_MAX || a.tile_pairs > INT32_MAX) return GS3D_ERR_OVERFLOW;
    if (groups >= (int64_t)1 << gs3d::kGroupBits || d.gx >= 0xFFFF || d.gy >= 0xFFFF) return GS3D_ERR_UNSUPPORTED;
    hipStream_t s = gs3d::as_stream(stream);
    if (a.group_pairs == 0 || a.tile_pairs == 0 || rows == 0) {
        gs3d::fill_u32(reinterpret_cast<uint32_t*>(a.ranges), 2 * tiles, 0u, s);
        if (a.caps && a.redo_list) gs3d::fill_u32(reinterpret_cast<uint32_t*>(a.redo_list), 1, 0u, s);
        return gs3d::launch_status("gs3d_bin_rows");
    }
    if (!a.centers || !a.radii || !a.order || !a.group_offsets || !a.ids || !scratch) return GS3D_ERR_ARGUMENT;
    if ((reinterpret_cast<uintptr_t>(a.ranges) & 7) || (reinterpret_cast<uintptr_t>(a.order) & 7) ||
        (reinterpret_cast<uintptr_t>(a.centers) & 7))
        return GS3D_ERR_ARGUMENT;
    if (scratch_bytes < gs3d_bin_rows_scratch_bytes(a.group_pairs, a.views, a.width, a.height, a.tile_mode))
        return GS3D_ERR_SCRATCH;
    const bool accu = a.tile_mode == GS3D_TILE_ACCUTILE;
    gs3d::BinScratch sc;
    gs3d::bin_scratch_bytes(a.group_pairs, groups, tiles, accu, &sc, scratch);
    const int64_t S = a.group_pairs;
    const int64_t chunks = gs3d::max_chunks_of(S, groups);
    const gs3d::RowGeometry geo{a.centers, a.conics, a.radii, a.tile_mode};
    const dim3 egrid(gs3d::blocks_for(rows, gs3d::kBinThreads)), eblock(gs3d::kBinThreads);
    const int group_bits = gs3d::bit_length(groups - 1 > 0 ? groups - 1 : 1);
    const uint64_t* items = sc.items;  // the sorted group items
    int status;
    if (accu) {
        if (!a.footprints || (reinterpret_cast<uintptr_t>(a.footprints) & 15)) return GS3D_ERR_ARGUMENT;
        const float4* fp = reinterpret_cast<const float4*>(a.footprints);
        if (d.gx <= 256 && d.gy <= 256)
            hipLaunchKernelGGL(gs3d::accutile_emit_kernel<true>, egrid, eblock, 0, s, a.order, a.group_offsets, rows,
                               geo, fp, a.n, d, S, sc.items, sc.masks);
        else
            hipLaunchKernelGGL(gs3d::accutile_emit_kernel<false>, egrid, eblock, 0, s, a.order, a.group_offsets, rows,
                               geo, fp, a.n, d, S, sc.items, sc.masks);
        status = gs3d::run_sort<uint64_t, uint64_t>(sc.items, sc.masks, S, group_bits, sc.sort, s);
    } else {
        if (!emitted) gs3d::emit_group_items(a, d, S, sc.items, s);
        if (group_bits <= gs3d::kOnePassBits) {
            // One 10-bit pass; its digit scan gives the group ranges, and the
            // chunk layout follows in the same workgroup.
            status = gs3d::run_sort_once<uint64_t>(sc.items, S, group_bits, sc.sort, (int)groups, sc.granges, s,
                                                   sc.chunk_base, sc.chunk_group);
            items = sc.items + S;
        } else {
            status = gs3d::run_sort<uint64_t, int32_t>(sc.items, nullptr, S, group_bits, sc.sort, s);
        }
    }
    if (status != GS3D_OK) return status;
    if (items == sc.items) {
        gs3d::fill_u32(reinterpret_cast<uint32_t*>(sc.granges), 2 * groups, 0u, s);
        hipLaunchKernelGGL(gs3d::tile_ranges_kernel<uint64_t>, dim3(gs3d::blocks_for(S, 256)), dim3(256), 0, s, items,
                           S, 0, gs3d::kGroupMask, sc.granges, groups);
        hipLaunchKernelGGL(gs3d::chunk_base_kernel, dim3(1), dim3(1024), 0, s, sc.granges, (int)groups,
                           sc.chunk_base);
        hipLaunchKernelGGL(gs3d::chunk_group_kernel, dim3(gs3d::blocks_for(chunks, 256)), dim3(256), 0, s,
                           sc.chunk_base, (int)groups, chunks, sc.chunk_group);
    }
    // The count pass writes every entry of the 64 * chunks table (zeros for
    // chunks beyond the groups' own).
    const dim3 pass_grid(gs3d::blocks_for(chunks, gs3d::kBinWaves));
    if (accu)
        hipLaunchKernelGGL((gs3d::group_pass_kernel<false, true>), pass_grid, dim3(gs3d::kBinThreads), 0, s, items,
                           sc.masks, sc.granges, sc.chunk_base, sc.chunk_group, (int)groups, chunks, d, sc.counts,
                           (const int32_t*)nullptr, (const int32_t*)nullptr, (int32_t*)nullptr, (int64_t)0,
                           (const int32_t*)nullptr, (const int32_t*)nullptr, (const int32_t*)nullptr,
                           (const int32_t*)nullptr, (unsigned long long*)nullptr, (int32_t*)nullptr);
    else
        hipLaunchKernelGGL((gs3d::group_pass_kernel<false, false>), pass_grid, dim3(gs3d::kBinThreads), 0, s, items,
                           (const uint64_t*)nullptr, sc.granges, sc.chunk_base, sc.chunk_group, (int)groups, chunks, d,
                           sc.counts, (const int32_t*)nullptr, (const int32_t*)nullptr, (int32_t*)nullptr, (int64_t)0,
                           (const int32_t*)nullptr, (const int32_t*)nullptr, (const int32_t*)nullptr,
                           (const int32_t*)nullptr, (unsigned long long*)nullptr, (int32_t*)nullptr);
    status = gs3d::run_scan<uint32_t, false>(sc.counts, 64 * chunks, sc.scanned, nullptr, sc.scan, s);
    if (status != GS3D_OK) return status;
    // (One workgroup computing totals, starts and ranges of up to 16K tiles
    // took 23-44 us against ~10 us for these three launches: each tile's
    // total is a chain of dependent loads.)
    hipLaunchKernelGGL(gs3d::tile_totals_kernel, dim3(gs3d::blocks_for(tiles, 256)), dim3(256), 0, s, sc.chunk_base,
                       sc.counts, sc.scanned, d, tiles, sc.totals);
    status = gs3d::run_scan<int32_t, false>(sc.totals, tiles, sc.starts, nullptr, sc.scan, s);
    if (status != GS3D_OK) return status;
    hipLaunchKernelGGL(gs3d::tile_ranges_from_totals_kernel, dim3(gs3d::blocks_for(tiles, 256)), dim3(256), 0, s,
                       sc.totals, sc.starts, tiles, a.ranges);
    return write_pass(a, sc, items, groups, chunks, d, a.caps, nullptr, nullptr, s);
}

// The id-write pass over binning state left in the scratch by bin_rows (the
// sorted group items at `items`, group ranges, chunk tables, scanned counts,
// tile starts): every tile's list, the first list_cap(caps[t]) entries of it
// with caps, only the tiles flagged in redo (whole lists; redo_count of
// them) with redo.
constexpr unsigned kRedoPassGrid = 1024;

template <int LISTS>
void launch_write_pass(const gs3d_bin_args& a, const BinScratch& sc, const uint64_t* items, int64_t groups,
                       int64_t chunks, const GridDims& d, const int32_t* caps, const int32_t* redo,
                       const int32_t* redo_count, hipStream_t s, unsigned long long* loaded = nullptr) {
    const bool accu = a.tile_mode == GS3D_TILE_ACCUTILE;
    const unsigned blocks = (unsigned)blocks_for(chunks, kBinWaves);
    const dim3 pass_grid(LISTS == 2 ? min(blocks, kRedoPassGrid) : blocks);
    // Buffer stores address the id list with 32-bit byte offsets.
    const bool buf = a.tile_pairs <= (int64_t)(0xFFFFFFFFu / 4);
#define GS3D_WRITE_PASS(M, B)                                                                                      \
    hipLaunchKernelGGL((group_pass_kernel<true, M, B, LISTS>), pass_grid, dim3(kBinThreads), 0, s, items,          \
                       M ? (const uint64_t*)sc.masks : nullptr, sc.granges, sc.chunk_base, sc.chunk_group,        \
                       (int)groups, chunks, d, sc.counts, sc.scanned, sc.starts, a.ids, a.tile_pairs, caps, redo, \
                       redo_count, sc.totals, loaded, LISTS == 1 ? a.redo_list : nullptr)
    if (accu) {
        if (buf)
            GS3D_WRITE_PASS(true, true);
        else
            GS3D_WRITE_PASS(true, false);
    } else {
        if (buf)
            GS3D_WRITE_PASS(false, true);
        else
            GS3D_WRITE_PASS(false, false);
    }
#undef GS3D_WRITE_PASS
}

int write_pass(const gs3d_bin_args& a, const BinScratch& sc, const uint64_t* items, int64_t groups, int64_t chunks,
               const GridDims& d, const int32_t* caps, const int32_t* redo, const int32_t* redo_count, hipStream_t s) {
    if (redo)
        launch_write_pass<2>(a, sc, items, groups, chunks, d, nullptr, redo, redo_count, s);
    else if (caps)
        launch_write_pass<1>(a, sc, items, groups, chunks, d, caps, nullptr, nullptr, s);
    else
        launch_write_pass<0>(a, sc, items, groups, chunks, d, nullptr, nullptr, nullptr, s);
    return launch_status("gs3d_bin_rows");
}

}  // namespace gs3d

extern "C" int gs3d_bin_rows(const gs3d_bin_args* args, void* scratch, size_t scratch_bytes, void* stream) {
    return gs3d::bin_rows(args, scratch, scratch_bytes, stream, false);
}

namespace gs3d {

// The binning state that gs3d_bin_rows / gs3d_bin_emitted_rows left in the
// scratch, for passes that follow them with the same arguments.
struct BinState {
    BinScratch sc;
    const uint64_t* items;  // the sorted group items
    int64_t groups, chunks;
    GridDims d;
};

// GS3D_OK with *state filled, 1 when the frame has no pairs (nothing to
// do), or an error status.
int bin_state(const gs3d_bin_args& a, void* scratch, size_t scratch_bytes, BinState* state) {
    if (a.n < 0 || a.views < 0 || a.width <= 0 || a.height <= 0 || a.group_pairs < 0 || a.tile_pairs < 0)
        return GS3D_ERR_ARGUMENT;
    const GridDims d = grid_dims(a.width, a.height);
    const int64_t rows = (int64_t)a.n * a.views;
    const int64_t groups = (int64_t)a.views * d.gpv, tiles = (int64_t)a.views * d.tpv;
    if (tiles == 0 || a.group_pairs == 0 || a.tile_pairs == 0 || rows == 0) return 1;
    if (rows > INT32_MAX || a.group_pairs > INT32_MAX || a.tile_pairs > INT32_MAX) return GS3D_ERR_OVERFLOW;
    if (groups >= (int64_t)1 << kGroupBits || d.gx >= 0xFFFF || d.gy >= 0xFFFF) return GS3D_ERR_UNSUPPORTED;
    if (!a.ids || !scratch) return GS3D_ERR_ARGUMENT;
    if (scratch_bytes < gs3d_bin_rows_scratch_bytes(a.group_pairs, a.views, a.width, a.height, a.tile_mode))
        return GS3D_ERR_SCRATCH;
    const bool accu = a.tile_mode == GS3D_TILE_ACCUTILE;
    bin_scratch_bytes(a.group_pairs, groups, tiles, accu, &state->sc, scratch);
    const int64_t S = a.group_pairs;
    const int group_bits = bit_length(groups - 1 > 0 ? groups - 1 : 1);
    // Where bin_rows left the sorted items: the second half after the
    // one-pass group sort, the first otherwise.
    state->items = !accu && group_bits <= kOnePassBits ? state->sc.items + S : state->sc.items;
    state->groups = groups;
    state->chunks = max_chunks_of(S, groups);
    state->d = d;
    return GS3D_OK;
}

}  // namespace gs3d

extern "C" int gs3d_bin_redo(const gs3d_bin_args* args, const int32_t* redo, const int32_t* redo_list,
                             void* scratch, size_t scratch_bytes, void* stream) {
    if (!args || !redo || !redo_list) return GS3D_ERR_ARGUMENT;
    gs3d::BinState st;
    const int status = gs3d::bin_state(*args, scratch, scratch_bytes, &st);
    if (status != GS3D_OK) return status == 1 ? GS3D_OK : status;
    return gs3d::write_pass(*args, st.sc, st.items, st.groups, st.chunks, st.d, nullptr, redo, redo_list,
                            gs3d::as_stream(stream));
}

extern "C" int gs3d_bin_capped_items(const gs3d_bin_args* args, void* scratch, size_t scratch_bytes,
                                     uint64_t* items_loaded, void* stream) {
    if (!args || !args->caps || !items_loaded || (reinterpret_cast<uintptr_t>(items_loaded) & 7))
        return GS3D_ERR_ARGUMENT;
    gs3d::BinState st;
    hipStream_t s = gs3d::as_stream(stream);
    gs3d::fill_u32(reinterpret_cast<uint32_t*>(items_loaded), 2, 0u, s);
    const int status = gs3d::bin_state(*args, scratch, scratch_bytes, &st);
    if (status != GS3D_OK) return status == 1 ? gs3d::launch_status("gs3d_bin_capped_items") : status;
    gs3d::launch_write_pass<3>(*args, st.sc, st.items, st.groups, st.chunks, st.d, args->caps, nullptr, nullptr, s,
                               reinterpret_cast<unsigned long long*>(items_loaded));
    return gs3d::launch_status("gs3d_bin_capped_items");
}

extern "C" int gs3d_emit_group_items(const gs3d_bin_args* args, void* scratch, size_t scratch_bytes, void* stream) {
    if (!args) return GS3D_ERR_ARGUMENT;
    const gs3d_bin_args& a = *args;
    if (a.n < 0 || a.views < 0 || a.width <= 0 || a.height <= 0 || a.group_pairs < 0) return GS3D_ERR_ARGUMENT;
    if (a.tile_mode == GS3D_TILE_ACCUTILE) return GS3D_ERR_UNSUPPORTED;
    if (gs3d::check_tile_mode(a.tile_mode, a.tile_mode == GS3D_TILE_RADIUS ? nullptr : a.conics) != GS3D_OK)
        return GS3D_ERR_ARGUMENT;
    const gs3d::GridDims d = gs3d::grid_dims(a.width, a.height);
    const int64_t rows = (int64_t)a.n * a.views;
    const int64_t groups = (int64_t)a.views * d.gpv;
    if (rows > INT32_MAX || a.group_pairs > INT32_MAX) return GS3D_ERR_OVERFLOW;
    if (groups >= (int64_t)1 << gs3d::kGroupBits || d.gx >= 0xFFFF || d.gy >= 0xFFFF) return GS3D_ERR_UNSUPPORTED;
    if (a.group_pairs == 0 || rows == 0 || groups == 0) return GS3D_OK;
    if (!a.centers || !a.radii || !a.order || !a.group_offsets || !scratch) return GS3D_ERR_ARGUMENT;
    if ((reinterpret_cast<uintptr_t>(a.order) & 7) || (reinterpret_cast<uintptr_t>(a.centers) & 7))
        return GS3D_ERR_ARGUMENT;
    if (scratch_bytes < gs3d_bin_rows_scratch_bytes(a.group_pairs, a.views, a.width, a.height, a.tile_mode))
        return GS3D_ERR_SCRATCH;
    gs3d::emit_group_items(a, d, a.group_pairs, reinterpret_cast<uint64_t*>(scratch), gs3d::as_stream(stream));
    return gs3d::launch_status("gs3d_emit_group_items");
}

extern "C" int gs3d_bin_emitted_rows(const gs3d_bin_args* args, void* scratch, size_t scratch_bytes, void* stream) {
    return gs3d::bin_rows(args, scratch, scratch_bytes, stream, true);
}

extern "C" int gs3d_pair_tiles(const int32_t* ranges, int64_t tile_count, uint32_t* tiles, int64_t count,
                               void* stream) {
    if (tile_count < 0 || count < 0) return GS3D_ERR_ARGUMENT;
    if (tile_count == 0 || count == 0) return GS3D_OK;
    if (!ranges || !tiles) return GS3D_ERR_ARGUMENT;
    if (tile_count > INT32_MAX) return GS3D_ERR_OVERFLOW;
    hipLaunchKernelGGL(gs3d::pair_tiles_kernel, dim3((unsigned)tile_count), dim3(256), 0, gs3d::as_stream(stream),
                       ranges, tile_count, tiles, count);
    return gs3d::launch_status("gs3d_pair_tiles");
}

extern "C" int gs3d_expand_keys(const uint32_t* sorted_tiles, const int32_t* ids, int64_t count, const float* depths,
                                int32_t n, int32_t tiles_per_view, uint64_t* keys, void* stream) {
    if (count < 0 || n < 0 || tiles_per_view <= 0) return GS3D_ERR_ARGUMENT;
    if (count == 0) return GS3D_OK;
    if (!sorted_tiles || !ids || !depths || !keys) return GS3D_ERR_ARGUMENT;
    hipLaunchKernelGGL(gs3d::expand_keys_kernel, dim3(gs3d::blocks_for(count, 256)), dim3(256), 0,
                       gs3d::as_stream(stream), sorted_tiles, ids, count, depths, n, tiles_per_view, keys);
    return gs3d::launch_status("gs3d_expand_keys");
}
