// Front-to-back alpha blending on 16x16 tiles and its reverse traversal.
//
// gs3d/render.py:36-208 (forward) and :211-356 (backward).  One 256-thread
// workgroup (four wave64 wavefronts, four pixel rows each) per tile; the
// tile's sorted Gaussians are staged in LDS in batches of 256 (centre, conic
// + opacity and the full blended channel vector), so the inner loop reads
// only LDS broadcasts.  A lane leaves the inner loop as soon as its pixel is
// done, so a wavefront stops when its 64 pixels are; the block stops at the
// next batch once all 256 are.
//
// Backward: every lane computes its pixel's contribution to the current
// Gaussian, the wavefront sums the contributions with DPP (lane 63 holds the
// sums) and lane 63 issues one atomic per gradient entry, instead of one per
// pixel as in the reference.  Only batches below the largest last
// contributor of the tile are visited.
#include "common.hpp"

namespace gs3d {

constexpr int kTile = 16;
constexpr int kRenderThreads = 256;

struct TileInfo {
    int view, px, py, first, last;
    bool inside;
    int64_t pix;
};

GS3D_DEV TileInfo tile_info(const gs3d_render_args& a) {
    const int gx = (a.width + kTile - 1) / kTile, gy = (a.height + kTile - 1) / kTile;
    const int per_view = gx * gy;
    const int tile = blockIdx.x;
    TileInfo t;
    t.view = tile / per_view;
    const int local = tile - t.view * per_view;
    const int ty = local / gx, tx = local - ty * gx;
    t.px = tx * kTile + (threadIdx.x & (kTile - 1));
    t.py = ty * kTile + (threadIdx.x >> 4);
    t.inside = t.px < a.width && t.py < a.height;
    t.pix = ((int64_t)t.view * a.height + t.py) * a.width + t.px;
    t.first = a.ranges[2 * (int64_t)tile];
    t.last = a.ranges[2 * (int64_t)tile + 1];
    return t;
}

// Stage one Gaussian's centre, conic and channel vector into LDS slot.
template <int CH>
GS3D_DEV void stage_gaussian(const gs3d_render_args& a, int view, int32_t g, int slot, float2* s_xy, float4* s_con,
                             float* s_feat) {
    const int64_t row = (int64_t)view * a.n + g;
    s_xy[slot] = reinterpret_cast<const float2*>(a.centers)[row];
    s_con[slot] = reinterpret_cast<const float4*>(a.conics)[row];
    float* dst = s_feat + slot * CH;
    const float* f = a.features + view * a.feat_view_stride + (int64_t)g * a.feat_stride;
    int c = 0;
    for (int k = 0; k < a.feat_channels; ++k) dst[c++] = f[k];
    if (a.extra_channels) {
        const float* e = a.extra + view * a.extra_view_stride + (int64_t)g * a.extra_stride;
        for (int k = 0; k < a.extra_channels; ++k) dst[c++] = e[k];
    }
    if (a.one_tail) dst[c++] = 1.0f;
}

// Gaussians staged per batch: 256 (one per thread) while the channel vectors
// fit the LDS budget, 128 for the widest vectors.
template <int CH>
struct Batch {
    static constexpr int size = CH <= 36 ? kRenderThreads : kRenderThreads / 2;
};

template <int CH>
__global__ __launch_bounds__(kRenderThreads) void render_fwd_kernel(gs3d_render_args a) {
    constexpr int B = Batch<CH>::size;
    __shared__ float2 s_xy[B];
    __shared__ float4 s_con[B];
    __shared__ float s_feat[B * CH];
    const TileInfo t = tile_info(a);
    const int D = a.feat_channels + a.extra_channels + (a.one_tail ? 1 : 0);
    const float fx = (float)t.px, fy = (float)t.py;
    float color[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) color[c] = 0.0f;
    float T = 1.0f;
    int contributor = 0, last_contributor = 0;
    bool done = !t.inside;
    for (int begin = t.first; begin < t.last; begin += B) {
        if (__syncthreads_count(!done) == 0) break;
        const int idx = begin + (int)threadIdx.x;
        if ((int)threadIdx.x < B && idx < t.last)
            stage_gaussian<CH>(a, t.view, a.ids[idx], threadIdx.x, s_xy, s_con, s_feat);
        __syncthreads();
        const int cnt = min(B, t.last - begin);
        for (int j = 0; j < cnt; ++j) {
            if (done) break;
            ++contributor;
            const float2 xy = s_xy[j];
            const float4 con = s_con[j];
            const float dx = xy.x - fx, dy = xy.y - fy;
            const float power = blend_power(con.x, con.y, con.z, dx, dy);
            if (!(power <= 0.0f)) continue;
            const float alpha = sel_min(0.99f, con.w * blend_exp(power));
            if (!(alpha >= 1.0f / 255.0f)) continue;
            const float next_t = T * (1.0f - alpha);
            if (next_t < 0.0001f) {
                done = true;
                continue;
            }
            const float w = alpha * T;
            const float* f = s_feat + j * CH;
#pragma unroll
            for (int c = 0; c < CH; ++c)
                if (c < D) color[c] = __builtin_fmaf(f[c], w, color[c]);
            T = next_t;
            last_contributor = contributor;
        }
    }
    if (t.inside) {
        float* out = a.image + t.pix * D;
        const float* bg = a.background ? a.background + t.view * a.background_view_stride : nullptr;
#pragma unroll
        for (int c = 0; c < CH; ++c)
            if (c < D) out[c] = __builtin_fmaf(T, (bg && c < a.feat_channels) ? bg[c] : 0.0f, color[c]);
        a.final_t[t.pix] = T;
        a.contributors[t.pix] = last_contributor;
    }
}

template <int CH, bool ABS>
__global__ __launch_bounds__(kRenderThreads) void render_bwd_kernel(gs3d_render_bwd_args b) {
    constexpr int B = Batch<CH>::size;
    __shared__ float2 s_xy[B];
    __shared__ float4 s_con[B];
    __shared__ int32_t s_id[B];
    __shared__ float s_feat[B * CH];
    __shared__ int s_max_last;
    const gs3d_render_args& a = b.fwd;
    const TileInfo t = tile_info(a);
    const int D = a.feat_channels + a.extra_channels + (a.one_tail ? 1 : 0);
    const int Dg = D - (a.one_tail ? 1 : 0);
    const float fx = (float)t.px, fy = (float)t.py;
    const int lane = lane_id();
    float grad[CH], accum[CH], last_color[CH];
    float T = 0.0f, T_final = 0.0f, bg_grad = 0.0f, last_alpha = 0.0f;
    int last_contributor = 0;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        grad[c] = 0.0f;
        accum[c] = 0.0f;
        last_color[c] = 0.0f;
    }
    if (threadIdx.x == 0) s_max_last = 0;
    if (t.inside) {
        T_final = a.final_t[t.pix];
        T = T_final;
        last_contributor = a.contributors[t.pix];
        const float* up = b.upstream + t.pix * D;
        const float* bg = a.background ? a.background + t.view * a.background_view_stride : nullptr;
#pragma unroll
        for (int c = 0; c < CH; ++c)
            if (c < D) {
                grad[c] = up[c];
                bg_grad += ((bg && c < a.feat_channels) ? bg[c] : 0.0f) * grad[c];
            }
    }
    __syncthreads();
    if (last_contributor > 0) atomicMax(&s_max_last, last_contributor);
    __syncthreads();
    const int max_last = min(s_max_last, t.last - t.first);
    for (int top = max_last; top > 0; top -= B) {
        __syncthreads();
        const int p = top - 1 - (int)threadIdx.x;
        if ((int)threadIdx.x < B && p >= 0) {
            const int32_t g = a.ids[t.first + p];
            s_id[threadIdx.x] = g;
            stage_gaussian<CH>(a, t.view, g, threadIdx.x, s_xy, s_con, s_feat);
        }
        __syncthreads();
        const int cnt = min(B, top);
        for (int j = 0; j < cnt; ++j) {
            const int pos = top - 1 - j;
            if (__ballot(t.inside && pos < last_contributor) == 0) continue;
            const float2 xy = s_xy[j];
            const float4 con = s_con[j];
            const float dx = xy.x - fx, dy = xy.y - fy;
            const float power = blend_power(con.x, con.y, con.z, dx, dy);
            float G = 0.0f, alpha = 0.0f;
            bool acc = t.inside && pos < last_contributor && power <= 0.0f;
            if (acc) {
                G = blend_exp(power);
                alpha = sel_min(0.99f, con.w * G);
                acc = alpha >= 1.0f / 255.0f;
            }
            if (__ballot(acc) == 0) continue;
            float gfeat[CH];
            float dcx = 0.0f, dcy = 0.0f, gk0 = 0.0f, gk1 = 0.0f, gk2 = 0.0f, gk3 = 0.0f;
#pragma unroll
            for (int c = 0; c < CH; ++c) gfeat[c] = 0.0f;
            if (acc) {
                T = T / (1.0f - alpha);
                const float* f = s_feat + j * CH;
                float grad_alpha = 0.0f;
#pragma unroll
                for (int c = 0; c < CH; ++c)
                    if (c < D) {
                        accum[c] = last_alpha * last_color[c] + (1.0f - last_alpha) * accum[c];
                        last_color[c] = f[c];
                        grad_alpha += (f[c] - accum[c]) * grad[c];
                        if (c < Dg) gfeat[c] = alpha * T * grad[c];
                    }
                grad_alpha = grad_alpha * T + (-T_final / (1.0f - alpha)) * bg_grad;
                last_alpha = alpha;
                const float gv = con.w * grad_alpha;
                const float gdx = G * dx, gdy = G * dy;
                dcx = gv * (-gdx * con.x - gdy * con.y);
                dcy = gv * (-gdy * con.z - gdx * con.y);
                gk0 = -0.5f * gdx * dx * gv;
                gk1 = -gdx * dy * gv;
                gk2 = -0.5f * gdy * dy * gv;
                gk3 = G * grad_alpha;
            }
            // Wavefront sums (lane 63) and one atomic per entry.
            const float s_dcx = wave_sum_to_lane63(dcx);
            const float s_dcy = wave_sum_to_lane63(dcy);
            const float s_k0 = wave_sum_to_lane63(gk0);
            const float s_k1 = wave_sum_to_lane63(gk1);
            const float s_k2 = wave_sum_to_lane63(gk2);
            const float s_k3 = wave_sum_to_lane63(gk3);
            float s_ax = 0.0f, s_ay = 0.0f;
            if (ABS) {
                s_ax = wave_sum_to_lane63(__builtin_fabsf(dcx));
                s_ay = wave_sum_to_lane63(__builtin_fabsf(dcy));
            }
            float s_f[CH];
#pragma unroll
            for (int c = 0; c < CH; ++c) s_f[c] = (c < Dg) ? wave_sum_to_lane63(gfeat[c]) : 0.0f;
            if (lane == 63) {
                const int32_t g = s_id[j];
                const int64_t row = (int64_t)t.view * a.n + g;
                float* gc = b.grad_centers + row * b.grad_centers_stride;
                atomicAdd(gc, s_dcx);
                atomicAdd(gc + 1, s_dcy);
                float* gk = b.grad_conics + row * b.grad_conics_stride;
                atomicAdd(gk, s_k0);
                atomicAdd(gk + 1, s_k1);
                atomicAdd(gk + 2, s_k2);
                atomicAdd(gk + 3, s_k3);
                if (ABS) {
                    float* ab = b.abs_centers + row * b.abs_stride;
                    atomicAdd(ab, s_ax);
                    atomicAdd(ab + 1, s_ay);
                }
                if (b.grad_features) {
                    float* gf = b.grad_features + t.view * b.grad_feat_view_stride + (int64_t)g * b.grad_feat_stride;
#pragma unroll
                    for (int c = 0; c < CH; ++c)
                        if (c < a.feat_channels) atomicAdd(gf + c, s_f[c]);
                }
                if (b.grad_extra) {
                    float* ge = b.grad_extra + t.view * b.grad_extra_view_stride + (int64_t)g * b.grad_extra_stride;
#pragma unroll
                    for (int c = 0; c < CH; ++c)
                        if (c >= a.feat_channels && c < Dg) atomicAdd(ge + (c - a.feat_channels), s_f[c]);
                }
            }
        }
    }
}

template <int CH>
int launch_fwd(const gs3d_render_args& a, unsigned blocks, hipStream_t s) {
    hipLaunchKernelGGL(render_fwd_kernel<CH>, dim3(blocks), dim3(kRenderThreads), 0, s, a);
    return launch_status("gs3d_render_fwd");
}

template <int CH>
int launch_bwd(const gs3d_render_bwd_args& b, unsigned blocks, hipStream_t s) {
    if (b.abs_centers)
        hipLaunchKernelGGL((render_bwd_kernel<CH, true>), dim3(blocks), dim3(kRenderThreads), 0, s, b);
    else
        hipLaunchKernelGGL((render_bwd_kernel<CH, false>), dim3(blocks), dim3(kRenderThreads), 0, s, b);
    return launch_status("gs3d_render_bwd");
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
    if (D > 64) return GS3D_ERR_UNSUPPORTED;  // widest compiled channel vector
    return GS3D_OK;
}

inline unsigned render_blocks(const gs3d_render_args& a) {
    const int64_t per_view = (int64_t)((a.width + kTile - 1) / kTile) * ((a.height + kTile - 1) / kTile);
    return (unsigned)(per_view * a.views);
}

}  // namespace gs3d

extern "C" int gs3d_render_fwd(const gs3d_render_args* args, void* stream) {
    if (!args) return GS3D_ERR_ARGUMENT;
    const gs3d_render_args& a = *args;
    int status = gs3d::check_render_args(a);
    if (status != GS3D_OK) return status;
    if (a.views == 0) return GS3D_OK;
    if (!a.image || !a.final_t || !a.contributors) return GS3D_ERR_ARGUMENT;
    const int D = a.feat_channels + a.extra_channels + (a.one_tail ? 1 : 0);
    const unsigned blocks = gs3d::render_blocks(a);
    hipStream_t s = gs3d::as_stream(stream);
    if (D <= 4) return gs3d::launch_fwd<4>(a, blocks, s);
    if (D <= 8) return gs3d::launch_fwd<8>(a, blocks, s);
    if (D <= 16) return gs3d::launch_fwd<16>(a, blocks, s);
    if (D <= 36) return gs3d::launch_fwd<36>(a, blocks, s);
    return gs3d::launch_fwd<64>(a, blocks, s);
}

extern "C" int gs3d_render_bwd(const gs3d_render_bwd_args* args, void* stream) {
    if (!args) return GS3D_ERR_ARGUMENT;
    const gs3d_render_bwd_args& b = *args;
    const gs3d_render_args& a = b.fwd;
    int status = gs3d::check_render_args(a);
    if (status != GS3D_OK) return status;
    if (a.views == 0) return GS3D_OK;
    if (!a.final_t || !a.contributors || !b.upstream || !b.grad_centers || !b.grad_conics) return GS3D_ERR_ARGUMENT;
    if (b.grad_centers_stride < 2 || b.grad_conics_stride < 4 || (b.abs_centers && b.abs_stride < 2))
        return GS3D_ERR_ARGUMENT;
    const int D = a.feat_channels + a.extra_channels + (a.one_tail ? 1 : 0);
    const unsigned blocks = gs3d::render_blocks(a);
    hipStream_t s = gs3d::as_stream(stream);
    if (D <= 4) return gs3d::launch_bwd<4>(b, blocks, s);
    if (D <= 8) return gs3d::launch_bwd<8>(b, blocks, s);
    if (D <= 16) return gs3d::launch_bwd<16>(b, blocks, s);
    if (D <= 36) return gs3d::launch_bwd<36>(b, blocks, s);
    return gs3d::launch_bwd<64>(b, blocks, s);
}
