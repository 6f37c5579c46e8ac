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
// LSD radix sort, 8-bit digits.  Per pass: per-tile digit histograms
// (digit-major [256][tiles]), one exclusive scan over them (the scatter base
// of every (digit, tile)), then a stable rank-and-scatter: each wavefront
// ranks its 1024 keys with ballot-based digit matching, the block orders the
// 4096 keys by digit in LDS and writes them out in digit runs.
// ---------------------------------------------------------------------------
constexpr int kSortThreads = 256;
constexpr int kSortItems = 16;
constexpr int kSortTile = kSortThreads * kSortItems;  // 4096 keys
constexpr int kRadix = 256;

GS3D_DEV uint32_t digit_of(uint64_t key, int shift, uint32_t mask) { return (uint32_t)(key >> shift) & mask; }

__global__ __launch_bounds__(kSortThreads) void sort_histogram_kernel(const uint64_t* __restrict__ keys, int64_t count,
                                                                      int shift, uint32_t mask,
                                                                      uint32_t* __restrict__ counts, int64_t tiles) {
    __shared__ uint32_t s_hist[kSortThreads / 64][kRadix];
    const int wave = threadIdx.x >> 6;
    for (int e = threadIdx.x; e < (kSortThreads / 64) * kRadix; e += kSortThreads) (&s_hist[0][0])[e] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kSortTile + wave * (kSortTile / 4) + lane_id();
#pragma unroll 4
    for (int k = 0; k < kSortItems; ++k) {
        const int64_t idx = base + k * 64;
        if (idx < count) atomicAdd(&s_hist[wave][digit_of(keys[idx], shift, mask)], 1u);
    }
    __syncthreads();
    for (int d = threadIdx.x; d < kRadix; d += kSortThreads) {
        uint32_t sum = 0;
#pragma unroll
        for (int w = 0; w < kSortThreads / 64; ++w) sum += s_hist[w][d];
        counts[(int64_t)d * tiles + blockIdx.x] = sum;
    }
}

__global__ __launch_bounds__(kSortThreads) void sort_scatter_kernel(
    const uint64_t* __restrict__ keys_in, const int32_t* __restrict__ vals_in, uint64_t* __restrict__ keys_out,
    int32_t* __restrict__ vals_out, int64_t count, int shift, uint32_t mask, int bits,
    const int32_t* __restrict__ scanned, int64_t tiles) {
    __shared__ uint64_t s_keys[kSortTile];
    __shared__ int32_t s_vals[kSortTile];
    __shared__ uint32_t s_wcnt[kSortThreads / 64][kRadix];
    __shared__ int32_t s_gbase[kRadix];
    __shared__ uint32_t s_wave_tot[kSortThreads / 64];
    const int wave = threadIdx.x >> 6, lane = lane_id();
    for (int e = threadIdx.x; e < (kSortThreads / 64) * kRadix; e += kSortThreads) (&s_wcnt[0][0])[e] = 0;
    const int64_t tile_base = (int64_t)blockIdx.x * kSortTile;
    const int64_t valid_count = min((int64_t)kSortTile, count - tile_base);
    uint64_t key[kSortItems];
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
            key[k] = 0;
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
    // Digit-major offsets: start of digit d in this tile, then each wave's
    // offset within the digit.
    {
        const int d = threadIdx.x;  // kSortThreads == kRadix
        uint32_t c[kSortThreads / 64];
        uint32_t tot = 0;
#pragma unroll
        for (int w = 0; w < kSortThreads / 64; ++w) {
            c[w] = s_wcnt[w][d];
            tot += c[w];
        }
        uint32_t block_total;
        __shared__ uint32_t s_scan_wave[kSortThreads / 64];
        const uint32_t start = block_exclusive_scan<kSortThreads>(tot, s_scan_wave, block_total);
        uint32_t run = start;
#pragma unroll
        for (int w = 0; w < kSortThreads / 64; ++w) {
            s_wcnt[w][d] = run;
            run += c[w];
        }
        s_gbase[d] = scanned[(int64_t)d * tiles + blockIdx.x] - (int32_t)start;
        (void)s_wave_tot;
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
#pragma unroll 4
    for (int j = 0; j < kSortItems; ++j) {
        const int p = j * kSortThreads + threadIdx.x;
        if (p < valid_count) {
            const uint64_t kk = s_keys[p];
            const int64_t dst = (int64_t)s_gbase[digit_of(kk, shift, mask)] + p;
            keys_out[dst] = kk;
            vals_out[dst] = s_vals[p];
        }
    }
}

// primitives/tiling.py:39-54.
// Tile ids at or beyond tile_count (0xFFFFFFFF included) are ignored.
__global__ void tile_ranges_kernel(const uint64_t* __restrict__ keys, int64_t count, int32_t* __restrict__ ranges,
                                   int64_t tile_count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const int64_t cur = (int64_t)(keys[i] >> 32);
    const bool cur_ok = cur < tile_count;
    if (i == 0) {
        if (cur_ok) ranges[2 * cur] = 0;
    } else {
        const int64_t prev = (int64_t)(keys[i - 1] >> 32);
        if (cur != prev) {
            if (prev < tile_count) ranges[2 * prev + 1] = (int32_t)i;
            if (cur_ok) ranges[2 * cur] = (int32_t)i;
        }
    }
    if (i == count - 1 && cur_ok) ranges[2 * cur + 1] = (int32_t)count;
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

extern "C" int gs3d_sort_pairs_u64(uint64_t* keys, int32_t* values, int64_t count, int32_t end_bit, void* scratch,
                                   size_t scratch_bytes, void* stream) {
    if (count < 0 || end_bit < 0 || end_bit > 64) return GS3D_ERR_ARGUMENT;
    if (count <= 1 || end_bit == 0) return GS3D_OK;
    if (count > INT32_MAX) return GS3D_ERR_OVERFLOW;
    if (!keys || !values || !scratch) return GS3D_ERR_ARGUMENT;
    if (scratch_bytes < gs3d_sort_scratch_bytes(count)) return GS3D_ERR_SCRATCH;
    gs3d::SortScratch sc;
    gs3d::sort_scratch_bytes(count, &sc, scratch);
    hipStream_t s = gs3d::as_stream(stream);
    const int64_t tiles = (count + gs3d::kSortTile - 1) / gs3d::kSortTile;
    uint64_t* kin = keys;
    int32_t* vin = values;
    uint64_t* kout = keys + count;
    int32_t* vout = values + count;
    int passes = 0;
    for (int shift = 0; shift < end_bit; shift += 8, ++passes) {
        const int bits = end_bit - shift < 8 ? end_bit - shift : 8;
        const uint32_t mask = (1u << bits) - 1u;
        hipLaunchKernelGGL(gs3d::sort_histogram_kernel, dim3((unsigned)tiles), dim3(gs3d::kSortThreads), 0, s, kin,
                           count, shift, mask, sc.counts, tiles);
        int status = gs3d::run_scan<uint32_t, false>(sc.counts, tiles * gs3d::kRadix, sc.scanned, nullptr,
                                                     sc.scan_scratch, s);
        if (status != GS3D_OK) return status;
        hipLaunchKernelGGL(gs3d::sort_scatter_kernel, dim3((unsigned)tiles), dim3(gs3d::kSortThreads), 0, s, kin, vin,
                           kout, vout, count, shift, mask, bits, sc.scanned, tiles);
        uint64_t* tk = kin;
        kin = kout;
        kout = tk;
        int32_t* tv = vin;
        vin = vout;
        vout = tv;
    }
    if (kin != keys) {
        hipMemcpyAsync(keys, kin, (size_t)count * sizeof(uint64_t), hipMemcpyDeviceToDevice, s);
        hipMemcpyAsync(values, vin, (size_t)count * sizeof(int32_t), hipMemcpyDeviceToDevice, s);
    }
    return gs3d::launch_status("gs3d_sort_pairs_u64");
}

extern "C" int gs3d_tile_ranges(const uint64_t* sorted_keys, int64_t count, int32_t* ranges, int64_t tile_count,
                                void* stream) {
    if (count < 0 || tile_count < 0) return GS3D_ERR_ARGUMENT;
    if (count == 0) return GS3D_OK;
    if (!sorted_keys || !ranges) return GS3D_ERR_ARGUMENT;
    hipLaunchKernelGGL(gs3d::tile_ranges_kernel, dim3(gs3d::blocks_for(count, 256)), dim3(256), 0,
                       gs3d::as_stream(stream), sorted_keys, count, ranges, tile_count);
    return gs3d::launch_status("gs3d_tile_ranges");
}
