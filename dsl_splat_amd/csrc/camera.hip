// Per-camera projection rows and pose VJP (one thread per camera).
//
// splatting/camera_kernels.py:11-66 (prepare_kernel) and :69-106
// (backward_kernel).  Products and sums stay unfused, as the reference
// kernels are compiled with fuse_fp disabled.
#include "common.hpp"

namespace gs3d {

__device__ bool finite_f(float v) { return __builtin_isfinite(v); }

// 4x4 inverse by cofactors (adjugate / determinant); returns the determinant.
__device__ float inverse44(const float* m, float* inv) {
    inv[0] = m[5] * m[10] * m[15] - m[5] * m[11] * m[14] - m[9] * m[6] * m[15] + m[9] * m[7] * m[14] +
             m[13] * m[6] * m[11] - m[13] * m[7] * m[10];
    inv[4] = -m[4] * m[10] * m[15] + m[4] * m[11] * m[14] + m[8] * m[6] * m[15] - m[8] * m[7] * m[14] -
             m[12] * m[6] * m[11] + m[12] * m[7] * m[10];
    inv[8] = m[4] * m[9] * m[15] - m[4] * m[11] * m[13] - m[8] * m[5] * m[15] + m[8] * m[7] * m[13] +
             m[12] * m[5] * m[11] - m[12] * m[7] * m[9];
    inv[12] = -m[4] * m[9] * m[14] + m[4] * m[10] * m[13] + m[8] * m[5] * m[14] - m[8] * m[6] * m[13] -
              m[12] * m[5] * m[10] + m[12] * m[6] * m[9];
    inv[1] = -m[1] * m[10] * m[15] + m[1] * m[11] * m[14] + m[9] * m[2] * m[15] - m[9] * m[3] * m[14] -
             m[13] * m[2] * m[11] + m[13] * m[3] * m[10];
    inv[5] = m[0] * m[10] * m[15] - m[0] * m[11] * m[14] - m[8] * m[2] * m[15] + m[8] * m[3] * m[14] +
             m[12] * m[2] * m[11] - m[12] * m[3] * m[10];
    inv[9] = -m[0] * m[9] * m[15] + m[0] * m[11] * m[13] + m[8] * m[1] * m[15] - m[8] * m[3] * m[13] -
             m[12] * m[1] * m[11] + m[12] * m[3] * m[9];
    inv[13] = m[0] * m[9] * m[14] - m[0] * m[10] * m[13] - m[8] * m[1] * m[14] + m[8] * m[2] * m[13] +
              m[12] * m[1] * m[10] - m[12] * m[2] * m[9];
    inv[2] = m[1] * m[6] * m[15] - m[1] * m[7] * m[14] - m[5] * m[2] * m[15] + m[5] * m[3] * m[14] +
             m[13] * m[2] * m[7] - m[13] * m[3] * m[6];
    inv[6] = -m[0] * m[6] * m[15] + m[0] * m[7] * m[14] + m[4] * m[2] * m[15] - m[4] * m[3] * m[14] -
             m[12] * m[2] * m[7] + m[12] * m[3] * m[6];
    inv[10] = m[0] * m[5] * m[15] - m[0] * m[7] * m[13] - m[4] * m[1] * m[15] + m[4] * m[3] * m[13] +
              m[12] * m[1] * m[7] - m[12] * m[3] * m[5];
    inv[14] = -m[0] * m[5] * m[14] + m[0] * m[6] * m[13] + m[4] * m[1] * m[14] - m[4] * m[2] * m[13] -
              m[12] * m[1] * m[6] + m[12] * m[2] * m[5];
    inv[3] = -m[1] * m[6] * m[11] + m[1] * m[7] * m[10] + m[5] * m[2] * m[11] - m[5] * m[3] * m[10] -
             m[9] * m[2] * m[7] + m[9] * m[3] * m[6];
    inv[7] = m[0] * m[6] * m[11] - m[0] * m[7] * m[10] - m[4] * m[2] * m[11] + m[4] * m[3] * m[10] +
             m[8] * m[2] * m[7] - m[8] * m[3] * m[6];
    inv[11] = -m[0] * m[5] * m[11] + m[0] * m[7] * m[9] + m[4] * m[1] * m[11] - m[4] * m[3] * m[9] -
              m[8] * m[1] * m[7] + m[8] * m[3] * m[5];
    inv[15] = m[0] * m[5] * m[10] - m[0] * m[6] * m[9] - m[4] * m[1] * m[10] + m[4] * m[2] * m[9] +
              m[8] * m[1] * m[6] - m[8] * m[2] * m[5];
    return m[0] * inv[0] + m[1] * inv[4] + m[2] * inv[8] + m[3] * inv[12];
}

// A 64-bit key of one camera's view matrix and intrinsics: each value
// rounded to 12 mantissa bits (so a pose that moves by a small optimiser
// step keeps its key), signed zeros merged, the words mixed by
// multiply-xorshift rounds.  Equal cameras get equal keys; distinct cameras
// share one only by a collision, which costs the caller no more than a stale
// hint.
__device__ uint64_t camera_key(const float* V, const float* K) {
    uint64_t h = 0x243F6A8885A308D3ull;
    auto mix = [&](float v) {
        uint32_t w = __float_as_uint(v);
        w = (w & 0x7FFFFFFFu) == 0u ? 0u : (w + 0x400u) & ~0x7FFu;
        h = (h ^ w) * 0xD6E8FEB86659FD93ull;
        h ^= h >> 32;
    };
    for (int e = 0; e < 16; ++e) mix(V[e]);
    for (int e = 0; e < 9; ++e) mix(K[e]);
    return h;
}

__global__ void camera_prepare_kernel(const float* __restrict__ views, const float* __restrict__ Ks, int count,
                                      int width, int height, int with_centers, float* __restrict__ full,
                                      float* __restrict__ inverse, float* __restrict__ centers,
                                      int32_t* __restrict__ errors, uint64_t* __restrict__ keys) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const float* K = Ks + 9 * i;
    const float* V = views + 16 * i;
    if (keys) keys[i] = camera_key(V, K);
    bool finite = true;
    for (int e = 0; e < 9; ++e) finite = finite && finite_f(K[e]);
    int error = 0;
    if (!finite || K[0] <= 0.0f || K[4] <= 0.0f)
        error = 2;
    else if (K[1] != 0.0f || K[3] != 0.0f || K[6] != 0.0f || K[7] != 0.0f || K[8] != 1.0f)
        error = 1;
    errors[i] = error;
    if (error) return;
    const float px = 2.0f * K[0] / (float)width;
    const float py = 2.0f * K[4] / (float)height;
    const float cx = 2.0f * K[2] / (float)width - 1.0f;
    const float cy = 2.0f * K[5] / (float)height - 1.0f;
    float* F = full + 16 * i;
    for (int col = 0; col < 4; ++col) {
        F[col] = px * V[col] + cx * V[8 + col];
        F[4 + col] = py * V[4 + col] + cy * V[8 + col];
        F[8 + col] = V[8 + col];
        F[12 + col] = V[8 + col];
    }
    if (with_centers) {
        float inv[16];
        const float det = inverse44(V, inv);
        if (det == 0.0f) {
            errors[i] = 3;
            return;
        }
        const float rdet = 1.0f / det;
        for (int e = 0; e < 16; ++e) inverse[16 * i + e] = inv[e] * rdet;
        for (int r = 0; r < 3; ++r) centers[3 * i + r] = inv[4 * r + 3] * rdet;
    }
}

__global__ void camera_backward_kernel(const float* __restrict__ Ks, const float* __restrict__ grad_full, int width,
                                       int height, const float* __restrict__ inverse,
                                       const float* __restrict__ grad_centers, int count,
                                       float* __restrict__ grad_views) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const float* K = Ks + 9 * i;
    const float px = 2.0f * K[0] / (float)width;
    const float py = 2.0f * K[4] / (float)height;
    const float cx = 2.0f * K[2] / (float)width - 1.0f;
    const float cy = 2.0f * K[5] / (float)height - 1.0f;
    const float* G = grad_full ? grad_full + 16 * i : nullptr;
    for (int row = 0; row < 4; ++row)
        for (int col = 0; col < 4; ++col) {
            float value = 0.0f;
            if (G) {
                if (row == 0)
                    value = px * G[col];
                else if (row == 1)
                    value = py * G[4 + col];
                else if (row == 2)
                    value = (cx * G[col] + cy * G[4 + col]) + G[8 + col] + G[12 + col];
            }
            if (grad_centers) {
                const float* inv = inverse + 16 * i;
                float vjp = 0.0f;
                for (int k = 0; k < 3; ++k) vjp += inv[4 * k + row] * grad_centers[3 * i + k];
                value -= vjp * inv[4 * col + 3];
            }
            grad_views[16 * i + 4 * row + col] = value;
        }
}

}  // namespace gs3d

extern "C" int gs3d_camera_prepare_keyed(const float* views, const float* Ks, int32_t count, int32_t width,
                                         int32_t height, int32_t with_centers, float* full, float* inverse,
                                         float* centers, int32_t* errors, uint64_t* keys, void* stream) {
    if (count < 0 || width <= 0 || height <= 0) return GS3D_ERR_ARGUMENT;
    if (count == 0) return GS3D_OK;
    if (!views || !Ks || !full || !errors || (with_centers && (!inverse || !centers))) return GS3D_ERR_ARGUMENT;
    if (reinterpret_cast<uintptr_t>(keys) & 7) return GS3D_ERR_ARGUMENT;
    hipLaunchKernelGGL(gs3d::camera_prepare_kernel, dim3(gs3d::blocks_for(count, 64)), dim3(64), 0,
                       gs3d::as_stream(stream), views, Ks, count, width, height, with_centers, full, inverse,
                       centers, errors, keys);
    return gs3d::launch_status("gs3d_camera_prepare");
}

extern "C" int gs3d_camera_prepare(const float* views, const float* Ks, int32_t count, int32_t width,
                                   int32_t height, int32_t with_centers, float* full, float* inverse,
                                   float* centers, int32_t* errors, void* stream) {
    return gs3d_camera_prepare_keyed(views, Ks, count, width, height, with_centers, full, inverse, centers, errors,
                                     nullptr, stream);
}

extern "C" int gs3d_camera_backward(const float* Ks, const float* grad_full, int32_t width, int32_t height,
                                    const float* inverse, const float* grad_centers, int32_t count,
                                    float* grad_views, void* stream) {
    if (count < 0 || width <= 0 || height <= 0) return GS3D_ERR_ARGUMENT;
    if (count == 0) return GS3D_OK;
    if (!Ks || !grad_views || (grad_centers && !inverse)) return GS3D_ERR_ARGUMENT;
    hipLaunchKernelGGL(gs3d::camera_backward_kernel, dim3(gs3d::blocks_for(count, 64)), dim3(64), 0,
                       gs3d::as_stream(stream), Ks, grad_full, width, height, inverse, grad_centers, count,
                       grad_views);
    return gs3d::launch_status("gs3d_camera_backward");
}
