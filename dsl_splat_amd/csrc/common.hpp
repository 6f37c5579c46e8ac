// Shared device helpers for the gfx950 gs3d kernels.
//
// Everything is compiled with -ffp-contract=off: a multiply followed by an
// add stays two roundings unless the code calls fmaf explicitly.  The
// projection, key and blend arithmetic below therefore reproduces a fixed
// operation sequence (integer outputs and the forward image are bit-exact
// against the CPU restatement that follows the same sequence).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gs3d_hip.h"

#define GS3D_DEV __device__ __forceinline__

namespace gs3d {

// Host side: record and translate a launch error (defined in abi.hip).
int launch_status(const char* where);
void set_error(const char* message);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline unsigned blocks_for(int64_t n, int threads) { return (unsigned)((n + threads - 1) / threads); }

// ---------------------------------------------------------------------------
// Branch-exact min/max/clamp: the C++ std::min/std::max selection rule
// (first operand unless the comparison picks the second), so NaN handling is
// the same on the host and the device.
// ---------------------------------------------------------------------------
// Streaming (non-temporal) stores for dense output streams written once
// (whole lines over a wavefront): they do not displace cached inputs, which
// speeds up the write-heavy projection, SH and group-emission kernels on this
// part.  Scattered or partial-line writes (radix-sort digit runs, per-tile id
// lists) keep plain stores, which the L2 merges: streaming them measured up
// to 1.9x slower.  GS3D_NT=0 turns every streaming store into a plain one.
#ifndef GS3D_NT
#define GS3D_NT 1
#endif
typedef float gs3d_f32x2 __attribute__((ext_vector_type(2)));
typedef float gs3d_f32x4 __attribute__((ext_vector_type(4)));
typedef int gs3d_i32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int gs3d_u32x4 __attribute__((ext_vector_type(4)));
template <class T>
GS3D_DEV void st_stream(T* p, T v) {
    if constexpr (GS3D_NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}
GS3D_DEV void st_stream(float2* p, float2 v) {
    if constexpr (GS3D_NT) __builtin_nontemporal_store(gs3d_f32x2{v.x, v.y}, reinterpret_cast<gs3d_f32x2*>(p));
    else *p = v;
}
GS3D_DEV void st_stream(float4* p, float4 v) {
    if constexpr (GS3D_NT)
        __builtin_nontemporal_store(gs3d_f32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<gs3d_f32x4*>(p));
    else *p = v;
}
GS3D_DEV void st_stream(int2* p, int2 v) {
    if constexpr (GS3D_NT) __builtin_nontemporal_store(gs3d_i32x2{v.x, v.y}, reinterpret_cast<gs3d_i32x2*>(p));
    else *p = v;
}
GS3D_DEV void st_stream(uint4* p, uint4 v) {
    if constexpr (GS3D_NT)
        __builtin_nontemporal_store(gs3d_u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<gs3d_u32x4*>(p));
    else *p = v;
}

GS3D_DEV float sel_max(float a, float b) { return (a < b) ? b : a; }
GS3D_DEV float sel_min(float a, float b) { return (b < a) ? b : a; }
GS3D_DEV float sel_clamp(float v, float lo, float hi) { return sel_min(sel_max(v, lo), hi); }

// torch.nn.functional.normalize of a quaternion, as the reference applies it
// before projection (inputs.py:252): q / max(|q|, 1e-12), the squares summed
// in component order.  Returns |q|.
GS3D_DEV float normalize_quat(float (&q)[4]) {
    const float norm = __builtin_sqrtf(((q[0] * q[0] + q[1] * q[1]) + q[2] * q[2]) + q[3] * q[3]);
    const float d = sel_max(norm, 1e-12f);
#pragma unroll
    for (int k = 0; k < 4; ++k) q[k] = q[k] / d;
    return norm;
}

// Gradient through normalize_quat: g <- (g - u (u.g)) / |q| for the unit
// quaternion u, or g / 1e-12 where the norm was clamped.
GS3D_DEV void normalize_quat_vjp(const float (&u)[4], float norm, float (&g)[4]) {
    if (norm > 1e-12f) {
        const float dot = ((u[0] * g[0] + u[1] * g[1]) + u[2] * g[2]) + u[3] * g[3];
#pragma unroll
        for (int k = 0; k < 4; ++k) g[k] = (g[k] - u[k] * dot) / norm;
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) g[k] = g[k] / 1e-12f;
    }
}

// ---------------------------------------------------------------------------
// exp for blending.  x = k ln2 + r, k = rint(x log2 e), two-constant
// Cody-Waite reduction (the high part of ln2 has 15 significant bits, so
// k*ln2_hi is exact for |k| < 512), degree-7 Taylor polynomial of e^r on
// |r| <= ln2/2 in Horner form, exact scaling by 2^k.  Inputs below -86 give 0
// (the result would be < 2^-124, three orders below the 1/255 threshold),
// which also keeps every intermediate normal.
// ---------------------------------------------------------------------------
GS3D_DEV float blend_exp(float x) {
    if (x < -86.0f) return 0.0f;
    const float k = __builtin_rintf(x * 1.44269502e+00f);
    float r = __builtin_fmaf(k, -6.93145752e-01f, x);
    r = __builtin_fmaf(k, -1.42860677e-06f, r);
    float p = 1.98412701e-04f;
    p = __builtin_fmaf(p, r, 1.38888892e-03f);
    p = __builtin_fmaf(p, r, 8.33333377e-03f);
    p = __builtin_fmaf(p, r, 4.16666679e-02f);
    p = __builtin_fmaf(p, r, 1.66666672e-01f);
    p = __builtin_fmaf(p, r, 5.00000000e-01f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)k);
}

// Gaussian exponent of the blend (gs3d/render.py:87-94 with the contraction
// fixed as fma(-0.5, fma(a dx, dx, (c dy) dy), -((b dx) dy))).
GS3D_DEV float blend_power(float a, float b, float c, float dx, float dy) {
    const float q = __builtin_fmaf(a * dx, dx, (c * dy) * dy);
    return __builtin_fmaf(-0.5f, q, -((b * dx) * dy));
}

// ---------------------------------------------------------------------------
// Wavefront (64-lane) reductions with DPP.  Within each row of 16 lanes a
// butterfly (quad_perm swaps, then row rotations by 4 and 8) leaves the row
// sum in every lane of the row; row_bcast15/row_bcast31 then fold the four
// row sums into lane 63.
// ---------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
GS3D_DEV float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, BANK_MASK, false));
}

GS3D_DEV float row_sum16(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x124>(v);  // row_ror:4
    v += dpp_f<0x128>(v);  // row_ror:8
    return v;
}

// Full wave sum; valid in lane 63.  All 64 lanes must be active.
GS3D_DEV float wave_sum_to_lane63(float v) {
    v = row_sum16(v);
    v += dpp_f<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_f<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

// The same wave sum of 32-bit integers (the radix sort's digit counts).
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
GS3D_DEV uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, BANK_MASK, false);
}

GS3D_DEV uint32_t wave_sum_u32_to_lane63(uint32_t v) {
    v += dpp_u<0xB1>(v);
    v += dpp_u<0x4E>(v);
    v += dpp_u<0x124>(v);
    v += dpp_u<0x128>(v);
    v += dpp_u<0x142, 0xA>(v);
    v += dpp_u<0x143, 0xC>(v);
    return v;
}

// Wave sum broadcast as a wave-uniform value.
GS3D_DEV float wave_sum(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_sum_to_lane63(v)), 63));
}

// Sums V per-lane values over the wavefront together.  Two permlane swap
// levels pair the values so that each add serves two of them (32-lane
// halves, then 16-lane rows), then a row butterfly finishes every row.  On
// return out[r] holds, in every lane of row q (lanes 16q..16q+15), the total
// of value 4r + {0, 2, 1, 3}[q]; rows whose index is V or more hold
// unspecified values.  All 64 lanes must be active.
template <int V>
GS3D_DEV void wave_sum_rows(const float (&v)[V], float (&out)[(V + 3) / 4]) {
    constexpr int W = (V + 1) / 2;
    constexpr int R = (V + 3) / 4;
    float w[W];
    if constexpr (V <= 16) {
        // Up to 16 entries (the 4- and 8-channel blend VJPs, the statistics
        // observer): the swaps as in-place instructions on copies the
        // wavefront sum owns, so both operands are consumed and no register
        // is copied out first.  The compiler cannot see the swap inside the
        // asm, so the wait states it needs after a VALU write of its operands
        // (and before its results are read) are spelled out as s_nop 1 on
        // both sides (3M Gaussians: 1789 -> 1756 us for the RGB blend VJP).
#pragma unroll
        for (int i = 0; i < W; ++i) {
            float a = v[2 * i];
            float b = (2 * i + 1 < V) ? v[2 * i + 1] : a;  // an unpaired value pairs with itself
            // a = [a lanes 0-31 | b lanes 0-31], b = [a lanes 32-63 | b lanes 32-63]
            asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
            w[i] = a + b;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float a = w[2 * r];
            float b = (2 * r + 1 < W) ? w[2 * r + 1] : a;
            // a = rows [a0 b0 a2 b2], b = rows [a1 b1 a3 b3]
            asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
            out[r] = row_sum16(a + b);
        }
    } else {
        // Wider sums keep the builtins: their copies cost less than the wait
        // states of this many inline swaps (36 channels: 1288 against 1448
        // us).
#pragma unroll
        for (int i = 0; i < W; ++i) {
            const float a = v[2 * i];
            const float b = (2 * i + 1 < V) ? v[2 * i + 1] : a;  // an unpaired value pairs with itself
            // first = [a lanes 0-31 | b lanes 0-31], second = [a lanes 32-63 | b lanes 32-63]
            const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
            w[i] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float a = w[2 * r];
            const float b = (2 * r + 1 < W) ? w[2 * r + 1] : a;
            // first = rows [a0 b0 a2 b2], second = rows [a1 b1 a3 b3]
            const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
            out[r] = row_sum16(__uint_as_float(p[0]) + __uint_as_float(p[1]));
        }
    }
}

// Index of the value whose total wave_sum_rows leaves in lane `lane` of
// out[lane & 15] (meaningful for (lane & 15) < R).
GS3D_DEV int wave_sum_rows_value(int lane) {
    const int q = lane >> 4;
    return 4 * (lane & 15) + ((q == 1) ? 2 : (q == 2) ? 1 : q);
}

GS3D_DEV int lane_id() { return __lane_id(); }

// Length of a tile's list that the id-write pass writes and the forward
// blend reads when the tile's previous frame stopped after `stop` entries
// (all its pixels terminated by then); a negative stop (the tile needed its
// whole list) gives no cap.
GS3D_DEV uint32_t list_cap(int32_t stop) {
    return stop < 0 ? 0xFFFFFFFFu : (uint32_t)stop + ((uint32_t)stop >> 2) + 128u;
}

// ---------------------------------------------------------------------------
// Tile rectangle of a projected Gaussian, splatting/geometry.py:22-30
// (truncating conversions, then clamping to the tile grid).
// ---------------------------------------------------------------------------
GS3D_DEV int trunc_clamp(float v, int hi) {
    int i = (int)v;
    i = i < 0 ? 0 : i;
    return i > hi ? hi : i;
}

GS3D_DEV int4 tile_rect(float cx, float cy, int radius, int gx, int gy) {
    const float r = (float)radius;
    int4 b;
    b.x = trunc_clamp((cx - r) / 16.0f, gx);
    b.y = trunc_clamp((cy - r) / 16.0f, gy);
    b.z = trunc_clamp(((cx + r) + 16.0f - 1.0f) / 16.0f, gx);
    b.w = trunc_clamp(((cy + r) + 16.0f - 1.0f) / 16.0f, gy);
    return b;
}

}  // namespace gs3d
