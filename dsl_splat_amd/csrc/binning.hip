// Tile binning: inclusive scan of tile counts, (tile << 32 | depth bits) key
// emission, stable LSD radix sort of (key, id) pairs and per-tile ranges.
//
// primitives/tiling.py:28-100 (float_bits, sort_key, identify_ranges,
// scan_counts, sort_tile_pairs) and splatting/binning.py:16-37, :71-117
// (duplicate, bin_and_sort).  All of it is integer work over HBM-resident
// arrays: coalesced loads, LDS-local reordering before every scatter, no
// matrix cores.
#include <climits>

#include "common.hpp"

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

// ---------------------------------------------------------------------------
// Scan (reduce-then-scan over 4096-element tiles).
// ---------------------------------------------------------------------------
template <class In>
__global__ __launch_bounds__(kScanThreads) void scan_reduce_kernel(const In* __restrict__ in, int64_t n,
                                                                   int64_t* __restrict__ partials) {
    __shared__ int64_t s_wave[kScanThreads / 64];
    const int64_t base = (int64_t)blockIdx.x * kScanTile;
    int64_t sum = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t idx = base + k * kScanThreads + threadIdx.x;
        if (idx < n) sum += (int64_t)in[idx];
    }
    int64_t total;
    block_exclusive_scan<kScanThreads>(sum, s_wave, total);
    if (threadIdx.x == 0) partials[blockIdx.x] = total;
}

// Exclusive scan of the tile partials in place (single block); writes the
// grand total.
__global__ __launch_bounds__(1024) void scan_partials_kernel(int64_t* __restrict__ partials, int64_t count,
                                                             int64_t* __restrict__ total_out) {
    __shared__ int64_t s_wave[1024 / 64];
    int64_t carry = 0;
    for (int64_t base = 0; base < count; base += 1024) {
        const int64_t idx = base + threadIdx.x;
        const int64_t v = idx < count ? partials[idx] : 0;
        int64_t total;
        const int64_t ex = block_exclusive_scan<1024>(v, s_wave, total);
        if (idx < count) partials[idx] = carry + ex;
        carry += total;
    }
    if (threadIdx.x == 0 && total_out) *total_out = carry;
}

// Per-tile scan with the tile's prefix; blocked layout per thread (16
// consecutive elements) so each thread writes a contiguous run.
template <class In, bool INCLUSIVE>
__global__ __launch_bounds__(kScanThreads) void scan_down_kernel(const In* __restrict__ in, int64_t n,
                                                                 const int64_t* __restrict__ partials,
                                                                 int32_t* __restrict__ out) {
    __shared__ int64_t s_wave[kScanThreads / 64];
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    int32_t vals[kScanItems];
    int64_t sum = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t idx = base + k;
        vals[k] = idx < n ? (int32_t)in[idx] : 0;
        sum += vals[k];
    }
    int64_t total;
    int64_t run = block_exclusive_scan<kScanThreads>(sum, s_wave, total) + partials[blockIdx.x];
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t idx = base + k;
        if (INCLUSIVE) run += vals[k];
        if (idx < n) out[idx] = (int32_t)run;
        if (!INCLUSIVE) run += vals[k];
    }
}

inline size_t scan_partials_bytes(int64_t n) {
    const int64_t tiles = (n + kScanTile - 1) / kScanTile;
    return (size_t)((tiles + 1) * sizeof(int64_t) + 255) & ~(size_t)255;
}

// Scratch layout: [partials (tiles int64)] [total int64 when total == NULL].
template <class In, bool INCLUSIVE>
int run_scan(const In* in, int64_t n, int32_t* out, int64_t* total, void* scratch, hipStream_t stream) {
    const int64_t tiles = (n + kScanTile - 1) / kScanTile;
    int64_t* partials = reinterpret_cast<int64_t*>(scratch);
    hipLaunchKernelGGL((scan_reduce_kernel<In>), dim3((unsigned)tiles), dim3(kScanThreads), 0, stream, in, n, partials);
    hipLaunchKernelGGL(scan_partials_kernel, dim3(1), dim3(1024), 0, stream, partials, tiles, total);
    hipLaunchKernelGGL((scan_down_kernel<In, INCLUSIVE>), dim3((unsigned)tiles), dim3(kScanThreads), 0, stream, in, n,
                       partials, out);
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

__global__ void fill_u32_kernel(uint32_t* p, int count, uint32_t value) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = value;
}

__global__ __launch_bounds__(kEmitThreads) void emit_small_kernel(gs3d_emit_args a, uint32_t* __restrict__ queue_count,
                                                                  int32_t* __restrict__ queue) {
    const int64_t rows = (int64_t)a.n * a.views;
    const int64_t r = (int64_t)blockIdx.x * kEmitThreads + threadIdx.x;
    if (r >= rows) return;
    const int radius = a.radii[r];
    if (radius <= 0) return;
    const int gx = (a.width + 15) / 16, gy = (a.height + 15) / 16;
    const float2 c = reinterpret_cast<const float2*>(a.centers)[r];
    const int4 rect = tile_rect(c.x, c.y, radius, gx, gy);
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
        const float2 c = reinterpret_cast<const float2*>(a.centers)[r];
        const int4 rect = tile_rect(c.x, c.y, a.radii[r], gx, gy);
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

// ---------------------------------------------------------------------------
// LSD radix sort of (key, int32 value) pairs, 8-bit digits, for 32- and
// 64-bit keys.  Per pass: per-tile digit histograms (digit-major
// [256][tiles]), one exclusive scan over them (the scatter base of every
// (digit, tile)), then a stable rank-and-scatter: each wavefront ranks its
// 1024 keys with ballot-based digit matching, the block orders its 4096 keys
// by digit in LDS and writes them out in digit runs (coalesced).
// ---------------------------------------------------------------------------
constexpr int kSortThreads = 256;
constexpr int kSortItems = 16;
constexpr int kSortTile = kSortThreads * kSortItems;  // 4096 keys
constexpr int kRadix = 256;

template <class K>
GS3D_DEV uint32_t digit_of(K key, int shift, uint32_t mask) { return (uint32_t)(key >> shift) & mask; }

template <class K>
__global__ __launch_bounds__(kSortThreads) void sort_histogram_kernel(const K* __restrict__ keys, int64_t count,
                                                                      int shift, uint32_t mask,
                                                                      uint32_t* __restrict__ counts, int64_t tiles) {
    __shared__ uint32_t s_hist[kSortThreads / 64][kRadix];
    const int wave = threadIdx.x >> 6;
    for (int e = threadIdx.x; e < (kSortThreads / 64) * kRadix; e += kSortThreads) (&s_hist[0][0])[e] = 0;
    const int64_t base = (int64_t)blockIdx.x * kSortTile + wave * (kSortTile / 4) + lane_id();
    K key[kSortItems];
#pragma unroll
    for (int k = 0; k < kSortItems; ++k) {
        const int64_t idx = base + k * 64;
        key[k] = idx < count ? keys[idx] : K(0);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kSortItems; ++k) {
        const int64_t idx = base + k * 64;
        if (idx < count) atomicAdd(&s_hist[wave][digit_of(key[k], shift, mask)], 1u);
    }
    __syncthreads();
    for (int d = threadIdx.x; d < kRadix; d += kSortThreads) {
        uint32_t sum = 0;
#pragma unroll
        for (int w = 0; w < kSortThreads / 64; ++w) sum += s_hist[w][d];
        counts[(int64_t)d * tiles + blockIdx.x] = sum;
    }
}

template <class K>
__global__ __launch_bounds__(kSortThreads) void sort_scatter_kernel(
    const K* __restrict__ keys_in, const int32_t* __restrict__ vals_in, K* __restrict__ keys_out,
    int32_t* __restrict__ vals_out, int64_t count, int shift, uint32_t mask, int bits,
    const int32_t* __restrict__ scanned, int64_t tiles) {
    __shared__ K s_keys[kSortTile];
    __shared__ int32_t s_vals[kSortTile];
    __shared__ uint32_t s_wcnt[kSortThreads / 64][kRadix];
    __shared__ int32_t s_gbase[kRadix];
    __shared__ uint32_t s_scan_wave[kSortThreads / 64];
    const int wave = threadIdx.x >> 6, lane = lane_id();
    for (int e = threadIdx.x; e < (kSortThreads / 64) * kRadix; e += kSortThreads) (&s_wcnt[0][0])[e] = 0;
    const int64_t tile_base = (int64_t)blockIdx.x * kSortTile;
    const int64_t valid_count = min((int64_t)kSortTile, count - tile_base);
    K key[kSortItems];
    int32_t val[kSortItems];
    uint32_t rank[kSortItems];
    const int64_t base = tile_base + wave * (kSortTile / 4) + lane;
#pragma unroll
    for (int k = 0; k < kSortItems; ++k) {
        const int64_t idx = base + k * 64;
        if (idx < count) {
            key[k] = keys_in[idx];
            val[k] = vals_in[idx];
        } else {
            key[k] = K(0);
            val[k] = 0;
        }
    }
    __syncthreads();
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
    for (int k = 0; k < kSortItems; ++k) {
        const int64_t idx = base + k * 64;
        rank[k] = 0;
        if (idx < count) {
            const uint32_t d = digit_of(key[k], shift, mask);
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
    {
        // Start of digit d in this tile's digit-sorted order, then each
        // wavefront's offset within the digit (kSortThreads == kRadix).
        const int d = threadIdx.x;
        uint32_t c[kSortThreads / 64];
        uint32_t tot = 0;
#pragma unroll
        for (int w = 0; w < kSortThreads / 64; ++w) {
            c[w] = s_wcnt[w][d];
            tot += c[w];
        }
        uint32_t block_total;
        const uint32_t start = block_exclusive_scan<kSortThreads>(tot, s_scan_wave, block_total);
        uint32_t run = start;
#pragma unroll
        for (int w = 0; w < kSortThreads / 64; ++w) {
            s_wcnt[w][d] = run;
            run += c[w];
        }
        s_gbase[d] = scanned[(int64_t)d * tiles + blockIdx.x] - (int32_t)start;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kSortItems; ++k) {
        const int64_t idx = base + k * 64;
        if (idx < count) {
            const uint32_t d = digit_of(key[k], shift, mask);
            const uint32_t pos = s_wcnt[wave][d] + rank[k];
            s_keys[pos] = key[k];
            s_vals[pos] = val[k];
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kSortItems; ++j) {
        const int p = j * kSortThreads + threadIdx.x;
        if (p < valid_count) {
            const K kk = s_keys[p];
            const int64_t dst = (int64_t)s_gbase[digit_of(kk, shift, mask)] + p;
            keys_out[dst] = kk;
            vals_out[dst] = s_vals[p];
        }
    }
}

struct SortScratch {
    uint32_t* counts;     // [256][tiles]
    int32_t* scanned;     // [256][tiles]
    void* scan_scratch;   // scan partials for 256*tiles entries
};

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

inline size_t sort_scratch_bytes(int64_t count, SortScratch* out, void* base) {
    const int64_t tiles = (count + kSortTile - 1) / kSortTile;
    const int64_t entries = tiles * kRadix;
    const size_t a = align256((size_t)entries * 4);
    const size_t b = align256((size_t)entries * 4);
    const size_t c = scan_partials_bytes(entries);
    if (out) {
        char* p = reinterpret_cast<char*>(base);
        out->counts = reinterpret_cast<uint32_t*>(p);
        out->scanned = reinterpret_cast<int32_t*>(p + a);
        out->scan_scratch = p + a + b;
    }
    return a + b + c;
}

// Sort keys[0:count)/values[0:count) on bits [0, end_bit) using
// keys[count:2count)/values[count:2count) as the ping-pong buffer.
template <class K>
int run_sort(K* keys, int32_t* values, int64_t count, int end_bit, void* scratch, hipStream_t s) {
    SortScratch sc;
    sort_scratch_bytes(count, &sc, scratch);
    const int64_t tiles = (count + kSortTile - 1) / kSortTile;
    K* kin = keys;
    int32_t* vin = values;
    K* kout = keys + count;
    int32_t* vout = values + count;
    for (int shift = 0; shift < end_bit; shift += 8) {
        const int bits = end_bit - shift < 8 ? end_bit - shift : 8;
        const uint32_t mask = (1u << bits) - 1u;
        hipLaunchKernelGGL((sort_histogram_kernel<K>), dim3((unsigned)tiles), dim3(kSortThreads), 0, s, kin, count,
                           shift, mask, sc.counts, tiles);
        const int status = run_scan<uint32_t, false>(sc.counts, tiles * kRadix, sc.scanned, nullptr, sc.scan_scratch, s);
        if (status != GS3D_OK) return status;
        hipLaunchKernelGGL((sort_scatter_kernel<K>), dim3((unsigned)tiles), dim3(kSortThreads), 0, s, kin, vin, kout,
                           vout, count, shift, mask, bits, sc.scanned, tiles);
        K* tk = kin;
        kin = kout;
        kout = tk;
        int32_t* tv = vin;
        vin = vout;
        vout = tv;
    }
    if (kin != keys) {
        hipMemcpyAsync(keys, kin, (size_t)count * sizeof(K), hipMemcpyDeviceToDevice, s);
        hipMemcpyAsync(values, vin, (size_t)count * sizeof(int32_t), hipMemcpyDeviceToDevice, s);
    }
    return launch_status("radix sort");
}

// ---------------------------------------------------------------------------
// Per-tile ranges (primitives/tiling.py:39-54).  Tile ids at or beyond
// tile_count (0xFFFFFFFF included) are ignored.
// ---------------------------------------------------------------------------
template <class K, int SHIFT>
__global__ void tile_ranges_kernel(const K* __restrict__ keys, int64_t count, int32_t* __restrict__ ranges,
                                   int64_t tile_count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const int64_t cur = (int64_t)(uint32_t)(keys[i] >> SHIFT);
    const bool cur_ok = cur < tile_count;
    if (i == 0) {
        if (cur_ok) ranges[2 * cur] = 0;
    } else {
        const int64_t prev = (int64_t)(uint32_t)(keys[i - 1] >> SHIFT);
        if (cur != prev) {
            if (prev < tile_count) ranges[2 * prev + 1] = (int32_t)i;
            if (cur_ok) ranges[2 * cur] = (int32_t)i;
        }
    }
    if (i == count - 1 && cur_ok) ranges[2 * cur + 1] = (int32_t)count;
}

// ---------------------------------------------------------------------------
// Depth-ordered binning.  Rows (view, Gaussian) are stably sorted by the
// bits of their depth; their tile counts are scanned in that order; pairs
// are emitted in that order with 32-bit tile keys; a stable sort on the tile
// id then leaves every tile's list in (depth bits, Gaussian id) order --
// the order of the stable sort of (tile << 32 | depth bits) keys over
// Gaussian-ordered pairs that the reference performs.
// ---------------------------------------------------------------------------
__global__ void depth_keys_kernel(const float* __restrict__ depths, int64_t rows, uint32_t* __restrict__ keys,
                                  int32_t* __restrict__ order) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows) return;
    keys[i] = __float_as_uint(depths[i]);
    order[i] = (int32_t)i;
}

__global__ void gather_counts_kernel(const int32_t* __restrict__ tiles, const int32_t* __restrict__ order,
                                     int64_t rows, int32_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < rows) out[i] = tiles[order[i]];
}

constexpr int kOrderedThreads = 256;

// One block per 256 consecutive ordered rows; the block's pairs form one
// contiguous output range that its threads fill with stride 256, locating
// each pair's row by binary search over the rows' inclusive ends in LDS.
__global__ __launch_bounds__(kOrderedThreads) void emit_ordered_kernel(gs3d_emit_ordered_args a) {
    __shared__ int32_t s_end[kOrderedThreads];
    __shared__ int32_t s_x0[kOrderedThreads], s_y0[kOrderedThreads], s_w[kOrderedThreads];
    __shared__ uint32_t s_tbase[kOrderedThreads];
    __shared__ int32_t s_id[kOrderedThreads];
    const int64_t rows = (int64_t)a.n * a.views;
    const int64_t r0 = (int64_t)blockIdx.x * kOrderedThreads;
    const int cnt = (int)min((int64_t)kOrderedThreads, rows - r0);
    const int gx = (a.width + 15) / 16, gy = (a.height + 15) / 16;
    const int t = threadIdx.x;
    if (t < cnt) {
        const int64_t i = r0 + t;
        const int64_t row = a.order[i];
        s_end[t] = a.offsets[i];
        const int radius = a.radii[row];
        int x0 = 0, y0 = 0, w = 1;
        if (radius > 0) {
            const float2 c = reinterpret_cast<const float2*>(a.centers)[row];
            const int4 rect = tile_rect(c.x, c.y, radius, gx, gy);
            x0 = rect.x;
            y0 = rect.y;
            w = max(rect.z - rect.x, 1);
        }
        const int64_t view = row / a.n;
        s_x0[t] = x0;
        s_y0[t] = y0;
        s_w[t] = w;
        s_tbase[t] = (uint32_t)(view * gx * gy);
        s_id[t] = (int32_t)(row - view * a.n);
    }
    __syncthreads();
    const int64_t S = r0 > 0 ? a.offsets[r0 - 1] : 0;
    const int64_t E = s_end[cnt - 1];
    for (int64_t p = S + t; p < E; p += kOrderedThreads) {
        int lo = 0, hi = cnt - 1;  // first j with s_end[j] > p
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (s_end[mid] > p)
                hi = mid;
            else
                lo = mid + 1;
        }
        const int64_t start = lo > 0 ? s_end[lo - 1] : S;
        const int local = (int)(p - start);
        const int w = s_w[lo];
        const int dy = local / w, dx = local - dy * w;
        a.tile_keys[p] = s_tbase[lo] + (uint32_t)((s_y0[lo] + dy) * gx + s_x0[lo] + dx);
        a.values[p] = s_id[lo];
    }
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

struct OrderScratch {
    uint32_t* keys;   // 2*rows
    int32_t* counts;  // rows
    void* sort;
    void* scan;
};

inline size_t order_scratch_bytes(int64_t rows, OrderScratch* out, void* base) {
    const size_t a = align256((size_t)rows * 2 * sizeof(uint32_t));
    const size_t b = align256((size_t)rows * sizeof(int32_t));
    const size_t c = align256(sort_scratch_bytes(rows, nullptr, nullptr));
    const size_t d = scan_partials_bytes(rows);
    if (out) {
        char* p = reinterpret_cast<char*>(base);
        out->keys = reinterpret_cast<uint32_t*>(p);
        out->counts = reinterpret_cast<int32_t*>(p + a);
        out->sort = p + a + b;
        out->scan = p + a + b + c;
    }
    return a + b + c + d;
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
    const int64_t rows = (int64_t)a.n * a.views;
    if (rows == 0) return GS3D_OK;
    if (!a.centers || !a.radii || !a.depths || !a.offsets || !a.keys || !a.values || !scratch)
        return GS3D_ERR_ARGUMENT;
    if (reinterpret_cast<uintptr_t>(a.centers) & 7) return GS3D_ERR_ARGUMENT;
    if (scratch_bytes < gs3d_emit_scratch_bytes(rows)) return GS3D_ERR_SCRATCH;
    const int64_t tiles_total = (int64_t)((a.width + 15) / 16) * ((a.height + 15) / 16) * a.views;
    if (tiles_total > 0xFFFFFFFFll) return GS3D_ERR_OVERFLOW;
    hipStream_t s = gs3d::as_stream(stream);
    uint32_t* queue_count = reinterpret_cast<uint32_t*>(scratch);
    int32_t* queue = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(scratch) + 256);
    hipLaunchKernelGGL(gs3d::fill_u32_kernel, dim3(1), dim3(64), 0, s, queue_count, 1, 0u);
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

extern "C" int gs3d_tile_ranges(const uint64_t* sorted_keys, int64_t count, int32_t* ranges, int64_t tile_count,
                                void* stream) {
    if (count < 0 || tile_count < 0) return GS3D_ERR_ARGUMENT;
    if (count == 0) return GS3D_OK;
    if (!sorted_keys || !ranges) return GS3D_ERR_ARGUMENT;
    hipLaunchKernelGGL((gs3d::tile_ranges_kernel<uint64_t, 32>), dim3(gs3d::blocks_for(count, 256)), dim3(256), 0,
                       gs3d::as_stream(stream), sorted_keys, count, ranges, tile_count);
    return gs3d::launch_status("gs3d_tile_ranges");
}

extern "C" int gs3d_tile_ranges_u32(const uint32_t* sorted_tiles, int64_t count, int32_t* ranges,
                                    int64_t tile_count, void* stream) {
    if (count < 0 || tile_count < 0) return GS3D_ERR_ARGUMENT;
    if (count == 0) return GS3D_OK;
    if (!sorted_tiles || !ranges) return GS3D_ERR_ARGUMENT;
    hipLaunchKernelGGL((gs3d::tile_ranges_kernel<uint32_t, 0>), dim3(gs3d::blocks_for(count, 256)), dim3(256), 0,
                       gs3d::as_stream(stream), sorted_tiles, count, ranges, tile_count);
    return gs3d::launch_status("gs3d_tile_ranges_u32");
}

extern "C" size_t gs3d_depth_order_scratch_bytes(int64_t rows) {
    return gs3d::order_scratch_bytes(rows < 0 ? 0 : rows, nullptr, nullptr);
}

extern "C" int gs3d_depth_order(const float* depths, const int32_t* tiles, int64_t rows, int32_t* order,
                                int32_t* offsets, int64_t* total, void* scratch, size_t scratch_bytes, void* stream) {
    if (rows < 0) return GS3D_ERR_ARGUMENT;
    if (rows == 0) return GS3D_OK;
    if (rows > INT32_MAX) return GS3D_ERR_OVERFLOW;
    if (!depths || !tiles || !order || !offsets || !scratch) return GS3D_ERR_ARGUMENT;
    if (scratch_bytes < gs3d_depth_order_scratch_bytes(rows)) return GS3D_ERR_SCRATCH;
    gs3d::OrderScratch sc;
    gs3d::order_scratch_bytes(rows, &sc, scratch);
    hipStream_t s = gs3d::as_stream(stream);
    const dim3 grid(gs3d::blocks_for(rows, 256)), block(256);
    hipLaunchKernelGGL(gs3d::depth_keys_kernel, grid, block, 0, s, depths, rows, sc.keys, order);
    // order holds 2*rows entries: [0, rows) sorted result, [rows, 2rows) ping-pong.
    int status = gs3d::run_sort<uint32_t>(sc.keys, order, rows, 32, sc.sort, s);
    if (status != GS3D_OK) return status;
    hipLaunchKernelGGL(gs3d::gather_counts_kernel, grid, block, 0, s, tiles, order, rows, sc.counts);
    status = gs3d::run_scan<int32_t, true>(sc.counts, rows, offsets, total, sc.scan, s);
    if (status != GS3D_OK) return status;
    return gs3d::launch_status("gs3d_depth_order");
}

extern "C" int gs3d_emit_ordered(const gs3d_emit_ordered_args* args, void* stream) {
    if (!args) return GS3D_ERR_ARGUMENT;
    const gs3d_emit_ordered_args& a = *args;
    if (a.n < 0 || a.views < 0 || a.width <= 0 || a.height <= 0) return GS3D_ERR_ARGUMENT;
    const int64_t rows = (int64_t)a.n * a.views;
    if (rows == 0) return GS3D_OK;
    if (!a.centers || !a.radii || !a.order || !a.offsets || !a.tile_keys || !a.values) return GS3D_ERR_ARGUMENT;
    if (reinterpret_cast<uintptr_t>(a.centers) & 7) return GS3D_ERR_ARGUMENT;
    const int64_t tiles_total = (int64_t)((a.width + 15) / 16) * ((a.height + 15) / 16) * a.views;
    if (tiles_total > 0xFFFFFFFFll) return GS3D_ERR_OVERFLOW;
    hipLaunchKernelGGL(gs3d::emit_ordered_kernel, dim3(gs3d::blocks_for(rows, gs3d::kOrderedThreads)),
                       dim3(gs3d::kOrderedThreads), 0, gs3d::as_stream(stream), a);
    return gs3d::launch_status("gs3d_emit_ordered");
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
