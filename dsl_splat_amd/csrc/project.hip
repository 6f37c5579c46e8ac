// EWA projection, SH0-3 colour and training metadata (forward), and the
// projection / SH VJP (backward), one thread per Gaussian looping over views.
//
// Forward: gs3d/projection.py:37-164 (screen_covariance + project),
// splatting/geometry.py:22-123, splatting/math.py:8-47, primitives/math.py
// :14-45, primitives/sh.py:7-79 (basis + evaluate), splatting/metadata.py
// :12-31 (_prepare).  Backward: gs3d/projection.py:198-285 (projection_loss
// reverse pass) with the custom adjoints of splatting/geometry.py:42-51, :61-71
// and splatting/math.py:13-28, primitives/sh.py:82-138, and the Torch
// "means - camera centre" VJP of gs3d/api.py:160-164.
//
// HBM layout: Gaussians are read once per launch (means/quats/scales/opacity
// rows plus the SH block) and every view's outputs are written as contiguous
// (views, N, ...) rows.  SH blocks (N, K, 3) are staged through LDS so that
// global loads and stores are fully coalesced; each thread then reads its
// row from LDS with an odd row pitch (conflict-free).
#include "common.hpp"
#include "footprint.hpp"

#include <type_traits>

namespace gs3d {

constexpr int kProjBlock = 128;

struct M3 {
    float m[3][3];
};

GS3D_DEV M3 transpose3(const M3& a) {
    M3 r;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) r.m[i][j] = a.m[j][i];
    return r;
}

// splatting/math.py:31-41: fma(a[r,2], b[2,c], fma(a[r,0], b[0,c], a[r,1]*b[1,c])).
GS3D_DEV M3 ref_matmul(const M3& a, const M3& b) {
    M3 r;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            r.m[i][j] = __builtin_fmaf(a.m[i][2], b.m[2][j], __builtin_fmaf(a.m[i][0], b.m[0][j], a.m[i][1] * b.m[1][j]));
    return r;
}

// splatting/math.py:44-47.
GS3D_DEV float point_row(const float* M, int r, const float* p) {
    const float xy = __builtin_fmaf(M[4 * r + 0], p[0], M[4 * r + 1] * p[1]);
    return __builtin_fmaf(M[4 * r + 2], p[2], xy) + M[4 * r + 3];
}

// primitives/math.py:33-45.
GS3D_DEV M3 glm_rotation(const float* q) {
    const float r = q[0], x = q[1], y = q[2], z = q[3];
    const float yy = y * y, zz = z * z;
    const float rz = r * z, xz = x * z, rx = r * x;
    const float d0 = yy + zz, d1 = __builtin_fmaf(x, x, zz), d2 = __builtin_fmaf(x, x, yy);
    M3 R;
    R.m[0][0] = 1.0f - (d0 + d0);
    R.m[0][1] = 2.0f * __builtin_fmaf(x, y, rz);
    R.m[0][2] = 2.0f * __builtin_fmaf(-r, y, xz);
    R.m[1][0] = 2.0f * __builtin_fmaf(x, y, -rz);
    R.m[1][1] = 1.0f - (d1 + d1);
    R.m[1][2] = 2.0f * __builtin_fmaf(y, z, rx);
    R.m[2][0] = 2.0f * __builtin_fmaf(r, y, xz);
    R.m[2][1] = 2.0f * __builtin_fmaf(y, z, -rx);
    R.m[2][2] = 1.0f - (d2 + d2);
    return R;
}

struct CovParts {
    float t[3];
    float limx, limy;
    M3 Sigma, J, W, Tm, X;
};

// a / b, correctly rounded; with APPROX a times the hardware reciprocal of b
// (about one ulp), for quantities that only enter gradients.
template <bool APPROX>
GS3D_DEV float quotient(float a, float b) {
    if constexpr (APPROX)
        return a * __builtin_amdgcn_rcpf(b);
    else
        return a / b;
}

// 3D covariance Sigma = M^T M with M = S R(q) (gs3d/projection.py:37-86):
// the same for every view, so the kernels form it once per Gaussian.
GS3D_DEV M3 covariance_3d(const float* q, const float* s) {
    const M3 R = glm_rotation(q);
    M3 S;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) S.m[i][j] = 0.0f;
    S.m[0][0] = s[0];
    S.m[1][1] = s[1];
    S.m[2][2] = s[2];
    const M3 M = ref_matmul(S, R);
    return ref_matmul(transpose3(M), M);
}

// gs3d/projection.py:37-86 for one view, from the Gaussian's Sigma.  APPROX
// (the VJP's recomputation): the divisions of t, J and nothing else are
// approximate -- the clamp limits stay exact, and the VJP takes its clamp
// decisions from exact quotients of its own.
template <bool APPROX = false>
GS3D_DEV void screen_covariance(const float* pos, const M3& Sigma, const float* V, int width, int height, float fx,
                                float fy, CovParts& st, float* cov) {
    st.limx = 1.3f * (float)width / (2.0f * fx);
    st.limy = 1.3f * (float)height / (2.0f * fy);
    st.t[0] = sel_clamp(quotient<APPROX>(pos[0], pos[2]), -st.limx, st.limx) * pos[2];
    st.t[1] = sel_clamp(quotient<APPROX>(pos[1], pos[2]), -st.limy, st.limy) * pos[2];
    st.t[2] = pos[2];
    st.Sigma = Sigma;
    const float* t = st.t;
    st.J.m[0][0] = quotient<APPROX>(fx, t[2]);
    st.J.m[0][1] = 0.0f;
    st.J.m[0][2] = 0.0f;
    st.J.m[1][0] = 0.0f;
    st.J.m[1][1] = quotient<APPROX>(fy, t[2]);
    st.J.m[1][2] = 0.0f;
    st.J.m[2][0] = quotient<APPROX>(-(fx * t[0]), t[2] * t[2]);
    st.J.m[2][1] = quotient<APPROX>(-(fy * t[1]), t[2] * t[2]);
    st.J.m[2][2] = 0.0f;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) st.W.m[i][j] = V[4 * j + i];
    st.Tm = ref_matmul(st.W, st.J);
    st.X = ref_matmul(transpose3(st.Tm), transpose3(st.Sigma));
    const M3 cov2 = ref_matmul(st.X, st.Tm);
    cov[0] = cov2.m[0][0] + 0.3f;
    cov[1] = cov2.m[1][0];
    cov[2] = cov2.m[1][1] + 0.3f;
}

// splatting/geometry.py:106-123: fp32 divide, fp64 viewport, one rounding.
GS3D_DEV void pixel_center(const float* mean, const float* P, int width, int height, float* out) {
    float clip[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) clip[r] = point_row(P, r, mean);
    const float inv_w = 1.0f / (clip[3] + 0.0000001f);
    const double nx = (double)(clip[0] * inv_w);
    const double ny = (double)(clip[1] * inv_w);
    out[0] = (float)(((nx + 1.0) * (double)width - 1.0) * 0.5);
    out[1] = (float)(((ny + 1.0) * (double)height - 1.0) * 0.5);
}

struct Footprint {
    float center[2];
    float conic[3];
    int radius, tiles;
    float depth;
};

// gs3d/projection.py:113-162 for one (Gaussian, view); false when culled.
GS3D_DEV bool project_one(const float* mean, const M3& Sigma, const float* V, const float* P,
                          float fx, float fy, int width, int height, float near_plane, float far_plane,
                          float radius_clip, Footprint& f) {
    float t4[3];
#pragma unroll
    for (int r = 0; r < 3; ++r) t4[r] = point_row(V, r, mean);
    if (t4[2] <= near_plane || t4[2] >= far_plane) return false;
    CovParts st;
    float cov[3];
    screen_covariance(t4, Sigma, V, width, height, fx, fy, st, cov);
    const float a = cov[0], b = cov[1], c = cov[2];
    const float det = a * c - b * b;
    if (det == 0.0f) return false;
    const float mid = 0.5f * (a + c);
    const int radius = (int)__builtin_ceilf(3.0f * __builtin_sqrtf(mid + __builtin_sqrtf(sel_max(0.1f, mid * mid - det))));
    if ((float)radius <= radius_clip) return false;
    float center[2];
    pixel_center(mean, P, width, height, center);
    const int4 rect = tile_rect(center[0], center[1], radius, (width + 15) / 16, (height + 15) / 16);
    const int count = (rect.z - rect.x) * (rect.w - rect.y);
    if (count == 0) return false;
    const float inv = 1.0f / (a * c - b * b);
    f.center[0] = center[0];
    f.center[1] = center[1];
    f.conic[0] = c * inv;
    f.conic[1] = -b * inv;
    f.conic[2] = a * inv;
    f.radius = radius;
    f.tiles = count;
    f.depth = t4[2];
    return true;
}

// ---------------------------------------------------------------------------
// SH basis (primitives/sh.py:7-41) with float32 constants, left-to-right
// products, and its analytic gradient.
// ---------------------------------------------------------------------------
GS3D_DEV float sh_basis(const float* u, int k) {
    const float x = u[0], y = u[1], z = u[2];
    switch (k) {
    case 0: return 0.28209479177387814f;
    case 1: return -0.4886025119029199f * y;
    case 2: return 0.4886025119029199f * z;
    case 3: return -0.4886025119029199f * x;
    case 4: return 1.0925484305920792f * x * y;
    case 5: return -1.0925484305920792f * y * z;
    case 6: return 0.31539156525252005f * (2.0f * z * z - x * x - y * y);
    case 7: return -1.0925484305920792f * x * z;
    case 8: return 0.5462742152960396f * (x * x - y * y);
    case 9: return -0.5900435899266435f * y * (3.0f * x * x - y * y);
    case 10: return 2.890611442640554f * x * y * z;
    case 11: return -0.4570457994644658f * y * (4.0f * z * z - x * x - y * y);
    case 12: return 0.3731763325901154f * z * (2.0f * z * z - 3.0f * x * x - 3.0f * y * y);
    case 13: return -0.4570457994644658f * x * (4.0f * z * z - x * x - y * y);
    case 14: return 1.445305721320277f * z * (x * x - y * y);
    default: return -0.5900435899266435f * x * (x * x - 3.0f * y * y);
    }
}

GS3D_DEV void sh_basis_grad(const float* u, int k, float* g) {
#pragma clang fp contract(fast)  // backward only: compared within a tolerance
    const float x = u[0], y = u[1], z = u[2];
    const float C1 = 0.4886025119029199f, C4 = 1.0925484305920792f, C6 = 0.31539156525252005f,
                C8 = 0.5462742152960396f, C9 = 0.5900435899266435f, C10 = 2.890611442640554f,
                C11 = 0.4570457994644658f, C12 = 0.3731763325901154f, C14 = 1.445305721320277f;
    g[0] = g[1] = g[2] = 0.0f;
    switch (k) {
    case 0: break;
    case 1: g[1] = -C1; break;
    case 2: g[2] = C1; break;
    case 3: g[0] = -C1; break;
    case 4: g[0] = C4 * y; g[1] = C4 * x; break;
    case 5: g[1] = -C4 * z; g[2] = -C4 * y; break;
    case 6: g[0] = C6 * (-2.0f * x); g[1] = C6 * (-2.0f * y); g[2] = C6 * (4.0f * z); break;
    case 7: g[0] = -C4 * z; g[2] = -C4 * x; break;
    case 8: g[0] = C8 * (2.0f * x); g[1] = C8 * (-2.0f * y); break;
    case 9: g[0] = -C9 * (6.0f * x * y); g[1] = -C9 * (3.0f * x * x - 3.0f * y * y); break;
    case 10: g[0] = C10 * y * z; g[1] = C10 * x * z; g[2] = C10 * x * y; break;
    case 11:
        g[0] = -C11 * (-2.0f * x * y);
        g[1] = -C11 * (4.0f * z * z - x * x - 3.0f * y * y);
        g[2] = -C11 * (8.0f * y * z);
        break;
    case 12:
        g[0] = C12 * (-6.0f * x * z);
        g[1] = C12 * (-6.0f * y * z);
        g[2] = C12 * (6.0f * z * z - 3.0f * x * x - 3.0f * y * y);
        break;
    case 13:
        g[0] = -C11 * (4.0f * z * z - 3.0f * x * x - y * y);
        g[1] = -C11 * (-2.0f * x * y);
        g[2] = -C11 * (8.0f * x * z);
        break;
    case 14: g[0] = C14 * (2.0f * x * z); g[1] = C14 * (-2.0f * y * z); g[2] = C14 * (x * x - y * y); break;
    default: g[0] = -C9 * (3.0f * x * x - 3.0f * y * y); g[1] = -C9 * (-6.0f * x * y); break;
    }
}

GS3D_DEV float length3(const float* d) { return __builtin_sqrtf(d[0] * d[0] + d[1] * d[1] + d[2] * d[2]); }

// primitives/sh.py:58-77 for one row; raw receives the pre-clamp value.
template <int DEG>
GS3D_DEV void sh_eval(const float* coef, const float* dir, bool visible, float* color, float* raw) {
    float value[3] = {0.0f, 0.0f, 0.0f};
    if (visible) {
        float unit[3] = {0.0f, 0.0f, 0.0f};
        if (DEG > 0) {
            const float len = sel_max(length3(dir), 1.0e-12f);
#pragma unroll
            for (int i = 0; i < 3; ++i) unit[i] = dir[i] / len;
        }
#pragma unroll
        for (int k = 0; k < (DEG + 1) * (DEG + 1); ++k) {
            const float b = sh_basis(unit, k);
#pragma unroll
            for (int ch = 0; ch < 3; ++ch) value[ch] = value[ch] + b * coef[3 * k + ch];
        }
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) value[ch] = value[ch] + 0.5f;
    }
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) {
        raw[ch] = value[ch];
        color[ch] = sel_max(value[ch], 0.0f);
    }
}

// primitives/sh.py:100-136 for one row.  grad_coef receives (DEG+1)^2 * 3
// values (added to it when ACC, which lets views accumulate in place).
template <int DEG, bool ACC>
GS3D_DEV void sh_backward(const float* coef, const float* dir, bool visible, const bool* active, const float* up,
                          float* grad_coef, float* grad_dir) {
    constexpr int KC = (DEG + 1) * (DEG + 1);
    grad_dir[0] = grad_dir[1] = grad_dir[2] = 0.0f;
    if (!ACC) {
#pragma unroll
        for (int e = 0; e < 3 * KC; ++e) grad_coef[e] = 0.0f;
    }
    if (!visible) return;
    float cg[3];
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) cg[ch] = active[ch] ? up[ch] : 0.0f;
    float unit[3] = {0.0f, 0.0f, 0.0f}, length = 1.0f;
    if (DEG > 0) {
        length = length3(dir);
        const float l = sel_max(length, 1.0e-12f);
#pragma unroll
        for (int i = 0; i < 3; ++i) unit[i] = dir[i] / l;
    }
    float ug[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < KC; ++k) {
        const float b = sh_basis(unit, k);
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) {
            if (ACC)
                grad_coef[3 * k + ch] += b * cg[ch];
            else
                grad_coef[3 * k + ch] = b * cg[ch];
        }
        if (DEG > 0) {
            float bg[3];
            sh_basis_grad(unit, k, bg);
            const float d = coef[3 * k] * cg[0] + coef[3 * k + 1] * cg[1] + coef[3 * k + 2] * cg[2];
#pragma unroll
            for (int i = 0; i < 3; ++i) ug[i] = ug[i] + d * bg[i];
        }
    }
    if (DEG > 0) {
        const float l = sel_max(length, 1.0e-12f);
#pragma unroll
        for (int i = 0; i < 3; ++i) grad_dir[i] = ug[i] / l;
        if (length >= 1.0e-12f) {
            const float f = (unit[0] * ug[0] + unit[1] * ug[1] + unit[2] * ug[2]) / length;
#pragma unroll
            for (int i = 0; i < 3; ++i) grad_dir[i] = grad_dir[i] - unit[i] * f;
        }
    }
}

// ---------------------------------------------------------------------------
// Forward projection of every view, one thread per Gaussian (the colours are
// evaluated by sh_rows_fwd_kernel in a second launch).
// ---------------------------------------------------------------------------
// Cameras whose rows (view 16, projection 16, fx, fy) a block stages in LDS:
// the per-view loop then reads them with LDS broadcasts instead of vector
// loads through the L1 (0.174 -> 0.168 ms at 4 views).  More cameras read
// them from global memory.
constexpr int kCamLds = 16;

// At most 64 VGPRs (8 wavefronts per SIMD): this kernel is bound by its
// output stream, and more wavefronts in flight keep more stores queued.
template <bool META>
__global__ __launch_bounds__(kProjBlock) __attribute__((amdgpu_waves_per_eu(8))) void project_fwd_kernel(gs3d_project_args a) {
    const int n = a.n;
    const int64_t i = (int64_t)blockIdx.x * kProjBlock + threadIdx.x;
    __shared__ float s_cam[kCamLds][34];
    const bool staged = a.views <= kCamLds;
    if (staged) {
        for (int e = threadIdx.x; e < a.views * 34; e += kProjBlock) {
            const int v = e / 34, k = e - v * 34;
            s_cam[v][k] = k < 16   ? a.view[16 * v + k]
                          : k < 32 ? a.projection[16 * v + k - 16]
                                   : a.intrinsics[9 * v + (k == 32 ? 0 : 4)];
        }
        __syncthreads();
    }
    if (i >= n) return;
    float mean[3], q[4], s[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) mean[k] = a.means[3 * i + k];
    const float4 qq = reinterpret_cast<const float4*>(a.quats)[i];
    q[0] = qq.x;
    q[1] = qq.y;
    q[2] = qq.z;
    q[3] = qq.w;
    if (a.normalize_quats) normalize_quat(q);
#pragma unroll
    for (int k = 0; k < 3; ++k) s[k] = a.scales[3 * i + k];
    const float opac = a.opacities[i];
    const M3 Sigma = covariance_3d(q, s);
    auto one = [&](int v, const float* V, const float* P, float fx, float fy) {
        Footprint f;
        const bool vis = project_one(mean, Sigma, V, P, fx, fy, a.width, a.height, a.near_plane, a.far_plane,
                                     a.radius_clip, f);
        const int64_t row = (int64_t)v * n + i;
        if (!vis) f = Footprint{{0.0f, 0.0f}, {0.0f, 0.0f, 0.0f}, 0, 0, 0.0f};
        st_stream(reinterpret_cast<float2*>(a.centers) + row, make_float2(f.center[0], f.center[1]));
        st_stream(reinterpret_cast<float4*>(a.conics) + row,
                make_float4(f.conic[0], f.conic[1], f.conic[2], vis ? opac : 0.0f));
        st_stream(a.radii + row, f.radius);
        st_stream(a.tiles + row, f.tiles);
        st_stream(a.depths + row, f.depth);
        if constexpr (META) {
            st_stream(reinterpret_cast<float2*>(a.means2d) + row, make_float2(f.center[0], f.center[1]));
            st_stream(a.meta_opacities + row, vis ? opac : 0.0f);
#pragma unroll
            for (int k = 0; k < 3; ++k) st_stream(a.meta_conics + 3 * row + k, f.conic[k]);
        }
    };
    if (staged) {
        for (int v = 0; v < a.views; ++v) one(v, &s_cam[v][0], &s_cam[v][16], s_cam[v][32], s_cam[v][33]);
    } else {
        for (int v = 0; v < a.views; ++v)
            one(v, a.view + 16 * v, a.projection + 16 * v, a.intrinsics[9 * v], a.intrinsics[9 * v + 4]);
    }
}

// ---------------------------------------------------------------------------
// Backward: two persistent grid-stride kernels over blocks of Gaussians, the
// projection VJP and the SH VJP, each with a modest register and LDS
// footprint.  Camera gradients (view rows 0-2, projection rows 0,1,3, SH
// camera centres) are reduced per wavefront with DPP each iteration into
// wave-private LDS accumulators and summed over the block once at the end
// (one atomic per block and entry).
// ---------------------------------------------------------------------------
constexpr int kMaxViewsCamLds = 16;

// One view's projection VJP.  The covariance part stops at the gradient of
// the 3D covariance Sigma: it is linear in that gradient, so the views' sum
// goes through covariance_vjp once per Gaussian.
struct VJP {
    float mean[3], opacity;
    M3 sigma;           // d loss / d Sigma
    float view[3][4];   // rows 0..2
    float proj[3][4];   // rows 0, 1, 3
};

// C = A*B: gA += gC B^T, gB += A^T gC.
GS3D_DEV void matmul_vjp(const M3& A, const M3& B, const M3& gC, M3& gA, M3& gB) {
#pragma clang fp contract(fast)
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            float sa = 0.0f, sb = 0.0f;
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                sa += gC.m[i][k] * B.m[j][k];
                sb += A.m[k][i] * gC.m[k][j];
            }
            gA.m[i][j] += sa;
            gB.m[i][j] += sb;
        }
}

GS3D_DEV M3 zero3() {
    M3 z;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) z.m[i][j] = 0.0f;
    return z;
}

GS3D_DEV void projection_vjp(const float* mean, const M3& Sigma, const float* V, const float* P,
                             int width, int height, float fx, float fy, const float* gc, const float* gk, VJP& g) {
    // Gradients are compared within a tolerance: products and sums here may
    // fuse (the recomputed forward quantities come from the shared helpers,
    // which keep the forward's rounding).
#pragma clang fp contract(fast)
    float pos[3];
#pragma unroll
    for (int r = 0; r < 3; ++r) pos[r] = point_row(V, r, mean);
    // Divisions that only scale gradients use the hardware reciprocal; the
    // clamp decisions below keep exact quotients, as in the forward.
    CovParts st;
    float cov[3];
    screen_covariance<true>(pos, Sigma, V, width, height, fx, fy, st, cov);
    g.opacity = gk[3];
    // splatting/geometry.py:61-71.
    const float a = cov[0], b = cov[1], c = cov[2];
    const float det = a * c - b * b;
    const float factor = __builtin_amdgcn_rcpf(det * det + 0.0000001f);
    const float x = gk[0], y = gk[1], z = gk[2];
    M3 gcov2 = zero3();
    gcov2.m[0][0] = factor * (-c * c * x + b * c * y + (det - a * c) * z);
    gcov2.m[1][0] = factor * (2.0f * b * c * x - (det + 2.0f * b * b) * y + 2.0f * a * b * z);
    gcov2.m[1][1] = factor * (-a * a * z + a * b * y + (det - a * c) * x);
    M3 gX = zero3(), gTm = zero3();
    matmul_vjp(st.X, st.Tm, gcov2, gX, gTm);
    M3 gTmT = zero3(), gSigmaT = zero3();
    matmul_vjp(transpose3(st.Tm), transpose3(st.Sigma), gX, gTmT, gSigmaT);
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) gTm.m[i][j] += gTmT.m[j][i];
    g.sigma = transpose3(gSigmaT);
    M3 gW = zero3(), gJ = zero3();
    matmul_vjp(st.W, st.J, gTm, gW, gJ);
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) g.view[r][cc] = 0.0f;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) g.view[j][i] += gW.m[i][j];
    const float* t = st.t;
    const float tz2 = t[2] * t[2];
    const float rz2 = __builtin_amdgcn_rcpf(tz2), rz3 = __builtin_amdgcn_rcpf(tz2 * t[2]);
    float gt[3];
    gt[0] = gJ.m[2][0] * (-fx * rz2);
    gt[1] = gJ.m[2][1] * (-fy * rz2);
    gt[2] = gJ.m[0][0] * (-fx * rz2) + gJ.m[1][1] * (-fy * rz2) + gJ.m[2][0] * (2.0f * fx * t[0] * rz3) +
            gJ.m[2][1] * (2.0f * fy * t[1] * rz3);
    // splatting/geometry.py:42-51: saturated x/y are constants.
    const float xr = pos[0] / pos[2], yr = pos[1] / pos[2];
    float gpos[3];
    gpos[0] = (xr >= -st.limx && xr <= st.limx) ? gt[0] : 0.0f;
    gpos[1] = (yr >= -st.limy && yr <= st.limy) ? gt[1] : 0.0f;
    gpos[2] = gt[2];
#pragma unroll
    for (int k = 0; k < 3; ++k) g.mean[k] = 0.0f;
#pragma unroll
    for (int r = 0; r < 3; ++r) {
#pragma unroll
        for (int cc = 0; cc < 3; ++cc) {
            g.mean[cc] += gpos[r] * V[4 * r + cc];
            g.view[r][cc] += gpos[r] * mean[cc];
        }
        g.view[r][3] += gpos[r];
    }
    // Centre path.
    float clip[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) clip[r] = point_row(P, r, mean);
    const float inv_w = __builtin_amdgcn_rcpf(clip[3] + 0.0000001f);
    const float gnx = gc[0] * (0.5f * (float)width);
    const float gny = gc[1] * (0.5f * (float)height);
    const float gclip[3] = {gnx * inv_w, gny * inv_w, -(gnx * clip[0] + gny * clip[1]) * inv_w * inv_w};
    const int prow[3] = {0, 1, 3};
#pragma unroll
    for (int r = 0; r < 3; ++r) {
#pragma unroll
        for (int cc = 0; cc < 3; ++cc) {
            g.mean[cc] += gclip[r] * P[4 * prow[r] + cc];
            g.proj[r][cc] = gclip[r] * mean[cc];
        }
        g.proj[r][3] = gclip[r];
    }
}

// Sigma = M^T M with M = S R(q): quaternion and scale gradients of a summed
// d loss / d Sigma (splatting/math.py:13-28 for the rotation).
GS3D_DEV void covariance_vjp(const float* q, const float* s, const M3& gSigma, float* gq, float* gs) {
#pragma clang fp contract(fast)
    const M3 R = glm_rotation(q);
    M3 M;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) M.m[i][j] = s[i] * R.m[i][j];
    M3 gMT = zero3(), gM = zero3();
    matmul_vjp(transpose3(M), M, gSigma, gMT, gM);
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) gM.m[i][j] += gMT.m[j][i];
    M3 gR;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            acc += gM.m[i][j] * R.m[i][j];
            gR.m[i][j] = s[i] * gM.m[i][j];
        }
        gs[i] = acc;
    }
    const float r = q[0], qx = q[1], qy = q[2], qz = q[3];
    const auto& G = gR.m;
    gq[0] = 2.0f * (qz * (G[0][1] - G[1][0]) + qy * (G[2][0] - G[0][2]) + qx * (G[1][2] - G[2][1]));
    gq[1] = 2.0f * (qy * (G[0][1] + G[1][0]) + qz * (G[0][2] + G[2][0]) + r * (G[1][2] - G[2][1])) -
            4.0f * qx * (G[1][1] + G[2][2]);
    gq[2] = 2.0f * (qx * (G[0][1] + G[1][0]) + r * (G[2][0] - G[0][2]) + qz * (G[1][2] + G[2][1])) -
            4.0f * qy * (G[0][0] + G[2][2]);
    gq[3] = 2.0f * (r * (G[0][1] - G[1][0]) + qx * (G[0][2] + G[2][0]) + qy * (G[1][2] + G[2][1])) -
            4.0f * qz * (G[0][0] + G[1][1]);
}

// Projection VJP, all views of a Gaussian per thread.  Held to 128 VGPRs
// (4 wavefronts per SIMD; 0.309 -> 0.255 ms against the uncapped 135).
template <bool CAM>
__global__ __launch_bounds__(kProjBlock) __attribute__((amdgpu_waves_per_eu(4))) void project_bwd_kernel(
    gs3d_project_bwd_args a) {
    // Wave-private camera accumulators: [wave][view][entry] (view and
    // projection rows; the SH camera centre is handled by sh_rows_bwd_kernel).
    __shared__ float s_cam[CAM ? kProjBlock / 64 : 1][kMaxViewsCamLds][24];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n = a.n;
    const int views = a.views;
    if constexpr (CAM) {
        for (int e = threadIdx.x; e < (kProjBlock / 64) * kMaxViewsCamLds * 24; e += kProjBlock)
            (&s_cam[0][0][0])[e] = 0.0f;
        // The loop above zeroes other wavefronts' slices too: every zero must
        // land before any wavefront's lane 63 adds into its slice.
        __syncthreads();
    }
    for (int64_t base = (int64_t)blockIdx.x * kProjBlock; base < n; base += (int64_t)gridDim.x * kProjBlock) {
        const int64_t i = base + threadIdx.x;
        const bool valid = i < n;
        // Lanes past the last Gaussian read row n - 1 and write nothing: no
        // load waits behind a per-lane branch (each view's radius and
        // gradients are loaded together).
        const int64_t ic = valid ? i : (int64_t)n - 1;
        float mean[3], q[4], s[3], qnorm = 1.0f;
#pragma unroll
        for (int k = 0; k < 3; ++k) mean[k] = a.means[3 * ic + k];
        const float4 qq = reinterpret_cast<const float4*>(a.quats)[ic];
        q[0] = qq.x;
        q[1] = qq.y;
        q[2] = qq.z;
        q[3] = qq.w;
        if (a.normalize_quats) qnorm = normalize_quat(q);
#pragma unroll
        for (int k = 0; k < 3; ++k) s[k] = a.scales[3 * ic + k];
        const M3 Sigma = covariance_3d(q, s);
        float gm[3] = {0, 0, 0}, gq[4] = {0, 0, 0, 0}, gs[3] = {0, 0, 0}, go = 0.0f;
        M3 gsigma = zero3();
        for (int v = 0; v < views; ++v) {
            const int64_t row = (int64_t)v * n + ic;
            const float* gcp = a.grad_centers + row * a.grad_centers_stride;
            const float* gkp = a.grad_conics + row * a.grad_conics_stride;
            const int radius = a.radii[row];
            const float gc[2] = {gcp[0], gcp[1]};
            const float gk[4] = {gkp[0], gkp[1], gkp[2], gkp[3]};
            // Keeps the gradient loads beside the radius's instead of inside
            // the branch below.
            asm volatile("" ::"v"(gc[0]), "v"(gc[1]), "v"(gk[0]), "v"(gk[1]), "v"(gk[2]), "v"(gk[3]));
            const bool vis = valid && radius > 0;
            VJP g;
            float2 screen = make_float2(0.0f, 0.0f);
            if (vis) {
                screen = make_float2(gc[0], gc[1]);
                projection_vjp(mean, Sigma, a.view + 16 * v, a.projection + 16 * v, a.width, a.height,
                               a.intrinsics[9 * v], a.intrinsics[9 * v + 4], gc, gk, g);
#pragma unroll
                for (int k = 0; k < 3; ++k) gm[k] += g.mean[k];
#pragma unroll
                for (int r = 0; r < 3; ++r)
#pragma unroll
                    for (int c = 0; c < 3; ++c) gsigma.m[r][c] += g.sigma.m[r][c];
                go += g.opacity;
            }
            if (a.screen_grad && valid) st_stream(reinterpret_cast<float2*>(a.screen_grad) + row, screen);
            if constexpr (CAM) {
                if (v < kMaxViewsCamLds) {
#pragma unroll
                    for (int r = 0; r < 3; ++r)
#pragma unroll
                        for (int cc = 0; cc < 4; ++cc) {
                            const float sv = wave_sum_to_lane63(vis ? g.view[r][cc] : 0.0f);
                            const float sp = wave_sum_to_lane63(vis ? g.proj[r][cc] : 0.0f);
                            if (lane == 63) {
                                s_cam[wave][v][4 * r + cc] += sv;
                                s_cam[wave][v][12 + 4 * r + cc] += sp;
                            }
                        }
                }
            }
        }
        if (valid) {
            covariance_vjp(q, s, gsigma, gq, gs);
            if (a.grad_means)
#pragma unroll
                for (int k = 0; k < 3; ++k) a.grad_means[3 * i + k] = gm[k];  // read again by the SH VJP
            if (a.grad_quats) {
                if (a.normalize_quats) normalize_quat_vjp(q, qnorm, gq);
                st_stream(reinterpret_cast<float4*>(a.grad_quats) + i, make_float4(gq[0], gq[1], gq[2], gq[3]));
            }
            if (a.grad_scales)
#pragma unroll
                for (int k = 0; k < 3; ++k) st_stream(a.grad_scales + 3 * i + k, gs[k]);
            if (a.grad_opacities) st_stream(a.grad_opacities + i, go);
        }
    }
    if constexpr (CAM) {
        __syncthreads();
        const int total = views * 24;
        for (int e = threadIdx.x; e < total; e += kProjBlock) {
            const int v = e / 24, k = e - v * 24;
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < kProjBlock / 64; ++w) sum += s_cam[w][v][k];
            if (k < 12) {
                if (a.grad_view) atomicAdd(a.grad_view + 16 * v + k, sum);
            } else {
                const int r = (k - 12) >> 2, c = (k - 12) & 3;
                const int prow = r == 2 ? 3 : r;
                if (a.grad_projection) atomicAdd(a.grad_projection + 16 * v + 4 * prow + c, sum);
            }
        }
    }
}

constexpr int kShPrefetch = 4;  // views whose per-view inputs are loaded up front
// Views per group of the SH VJP: 2 keeps its registers at 3 wavefronts per
// SIMD (0.300 ms against 0.348 with 4 and 0.334 with 1).
constexpr int kShGroup = 2;

constexpr int kShRowBlock = 256;
// A wavefront's 64 rows of RF contiguous floats (16-byte aligned, RF a
// multiple of 4) between global memory and its LDS slice, where rows have the
// odd pitch RF + 1 (per-lane row reads are then free of bank conflicts).
// Every lane issues all of its float4 accesses before the first LDS write
// (one memory latency per copy); rows beyond `rows` are not touched.
template <int RF>
GS3D_DEV void rows_to_lds(float* lds, const float* glob, int rows) {
    static_assert(RF % 4 == 0, "float4 rows");
    constexpr int IT = RF / 4;  // float4s per lane for 64 rows
    const int lane = lane_id();
    const int limit = rows * (RF / 4);
    float4 v[IT];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int e4 = it * 64 + lane;
        if (e4 < limit) v[it] = reinterpret_cast<const float4*>(glob)[e4];
    }
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int e4 = it * 64 + lane;
        if (e4 < limit) {
            const int e = 4 * e4;
            float* l = lds + e + e / RF;
            l[0] = v[it].x;
            l[1] = v[it].y;
            l[2] = v[it].z;
            l[3] = v[it].w;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

template <int RF>
GS3D_DEV void lds_to_rows(const float* lds, float* glob, int rows) {
    static_assert(RF % 4 == 0, "float4 rows");
    constexpr int IT = RF / 4;
    const int lane = lane_id();
    const int limit = rows * (RF / 4);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int e4 = it * 64 + lane;
        if (e4 < limit) {
            const int e = 4 * e4;
            const float* l = lds + e + e / RF;
            st_stream(reinterpret_cast<float4*>(glob) + e4, make_float4(l[0], l[1], l[2], l[3]));
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// Row access modes of the SH kernels: per-lane scalar or float4 accesses,
// or rows staged through a wavefront's LDS slice (pitch E + 1).
enum ShRows : int { kRowsScalar = 0, kRowsFloat4 = 1, kRowsStaged = 2 };

// Colours of every view (primitives/sh.py:58-77 per row, sh_eval's order and
// rounding), one thread per Gaussian with its 3 * (DEG + 1)^2 coefficients in
// registers, loaded as float4 when VEC (rows 16-byte aligned, E a multiple
// of 4).  Runs after
// the projection kernel, whose radii mark the visible rows.
// Capped at 80 VGPRs (six wavefronts per SIMD; degree 3 needs 83 uncapped).
template <int DEG, bool VEC>
__global__ __launch_bounds__(kShRowBlock) __attribute__((amdgpu_waves_per_eu(6))) void sh_rows_fwd_kernel(gs3d_project_args a) {
    constexpr int KC = (DEG + 1) * (DEG + 1);
    const int64_t n = a.n;
    const int64_t i = (int64_t)blockIdx.x * kShRowBlock + threadIdx.x;
    const bool valid = i < n;
    const int views = a.views;
    const int64_t rf = (int64_t)a.sh_rows * 3;
    // Lanes past the last Gaussian load row n - 1 and store nothing: no load
    // sits behind a per-lane branch, so each step's loads are in flight
    // together.
    const int64_t ic = valid ? i : n - 1;
    float mean[3] = {0.0f, 0.0f, 0.0f};
    if (DEG > 0) {
#pragma unroll
        for (int k = 0; k < 3; ++k) mean[k] = a.means[3 * ic + k];
    }
    int pre_radius[kShPrefetch];
#pragma unroll
    for (int p = 0; p < kShPrefetch; ++p) pre_radius[p] = p < views ? a.radii[(int64_t)p * n + ic] : 0;
    float cf[3 * KC];
    for (int v = 0; v < views; ++v) {
        if (v == 0 || a.sh_view_stride != 0) {
            const float* src = a.sh + v * a.sh_view_stride + ic * rf;
            if constexpr (VEC && (3 * KC) % 4 == 0) {
#pragma unroll
                for (int e = 0; e < 3 * KC; e += 4) {
                    const float4 q = reinterpret_cast<const float4*>(src)[e >> 2];
                    cf[e] = q.x;
                    cf[e + 1] = q.y;
                    cf[e + 2] = q.z;
                    cf[e + 3] = q.w;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 3 * KC; ++e) cf[e] = src[e];
            }
        }
        const int64_t row = (int64_t)v * n + i;
        int radius = 0;
#pragma unroll
        for (int p = 0; p < kShPrefetch; ++p)
            if (v == p) radius = pre_radius[p];
        if (v >= kShPrefetch) radius = a.radii[(int64_t)v * n + ic];
        float dir[3] = {0.0f, 0.0f, 0.0f};
        if (DEG > 0) {
#pragma unroll
            for (int k = 0; k < 3; ++k) dir[k] = mean[k] - a.camera_centers[3 * v + k];
        }
        float color[3], raw[3];
        sh_eval<DEG>(cf, dir, radius > 0, color, raw);
        if (valid) {
#pragma unroll
            for (int c = 0; c < 3; ++c) st_stream(a.colors + 3 * row + c, color[c]);
        }
    }
}

// f(std::integral_constant<int, K>) for K = 0 .. N-1, unrolled at compile time.
template <int N, int K = 0, class F>
GS3D_DEV void static_for(F&& f) {
    if constexpr (K < N) {
        f(std::integral_constant<int, K>{});
        static_for<N, K + 1>(f);
    }
}

// Hides a value from the optimiser, so that expressions of it are evaluated
// again rather than kept live from an earlier use.
GS3D_DEV float opaque(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

// Adds (or, when !ACC, writes) COUNT gradient values at dst + BASE; float4
// accesses when VEC and the group is a whole 16-byte-aligned run of 12.
template <bool VEC, int BASE, int COUNT>
GS3D_DEV void put_sh_grads(float* dst, bool acc, const float* g) {
    if constexpr (VEC && COUNT == 12 && BASE % 4 == 0) {
        float4* d4 = reinterpret_cast<float4*>(dst + BASE);
#pragma unroll
        for (int q = 0; q < 3; ++q) {
            float4 v = make_float4(g[4 * q], g[4 * q + 1], g[4 * q + 2], g[4 * q + 3]);
            if (acc) {
                const float4 o = d4[q];
                v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
            }
            d4[q] = v;
        }
    } else {
#pragma unroll
        for (int e = 0; e < COUNT; ++e) dst[BASE + e] = acc ? dst[BASE + e] + g[e] : g[e];
    }
}

// SH VJP of every view (primitives/sh.py:100-136 per row), one thread per
// Gaussian with its E = 3 * (DEG + 1)^2 coefficients in registers, its rows
// read and written as MODE says (staged: coalesced copies through the
// wavefront's LDS slice, which also holds the gradient rows until they are
// stored).  Views are taken kShGroup at a time (one at a
// time for per-view coefficients): the clamp masks and directions of the
// group first, then one pass over the coefficient index that forms each
// coefficient's gradient over the group's views and stores it at once, so
// no accumulator per coefficient stays live; groups after the first add to
// the stored rows.  The direction gradients are added to grad_means (after
// project_bwd_kernel wrote it); with CAM the camera-centre gradients are
// reduced per wavefront into LDS accumulators.
template <int DEG, bool CAM, int MODE>
__global__ __launch_bounds__(kShRowBlock) void sh_rows_bwd_kernel(gs3d_project_bwd_args a) {
    constexpr int KC = (DEG + 1) * (DEG + 1);
    constexpr int E = 3 * KC;
    constexpr int U = kShGroup;
    constexpr bool vec = MODE == kRowsFloat4 && E % 4 == 0;
    constexpr bool staged = MODE == kRowsStaged && E % 4 == 0;
    constexpr int PITCH = E + 1;  // odd: per-lane row accesses are free of bank conflicts
    __shared__ float s_cam[CAM ? kShRowBlock / 64 : 1][kMaxViewsCamLds][3];
    __shared__ float s_stage[staged ? kShRowBlock / 64 : 1][staged ? 64 * PITCH : 1];
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    if constexpr (CAM) {
        for (int e = threadIdx.x; e < (kShRowBlock / 64) * kMaxViewsCamLds * 3; e += kShRowBlock)
            (&s_cam[0][0][0])[e] = 0.0f;
        __syncthreads();
    }
    const int64_t n = a.n;
    const int views = a.views;
    const bool per_view = a.sh_view_stride != 0;
    const int step = per_view ? 1 : U;
    const int64_t rf = (int64_t)a.sh_rows * 3;
    const int64_t g0 = (int64_t)blockIdx.x * kShRowBlock + (threadIdx.x & ~63);  // the wavefront's first row
    const int64_t i = g0 + lane;
    const bool valid = i < n;
    const int rows_here = (int)max((int64_t)0, min((int64_t)64, n - g0));
    float* stage = s_stage[staged ? wave : 0];
    float* const row_lds = stage + lane * PITCH;
    // Loads use clamped indices (row n - 1, the group's last view) and their
    // values are selected afterwards: a guarded load is a branch that waits
    // for its data, so every load of a step is in flight at once.
    const int64_t ic = valid ? i : n - 1;
    float mean[3] = {0.0f, 0.0f, 0.0f}, gm_old[3] = {0.0f, 0.0f, 0.0f}, gm[3] = {0.0f, 0.0f, 0.0f};
    if (DEG > 0) {
#pragma unroll
        for (int k = 0; k < 3; ++k) mean[k] = a.means[3 * ic + k];
        if (a.grad_means) {
#pragma unroll
            for (int k = 0; k < 3; ++k) gm_old[k] = a.grad_means[3 * ic + k];
        }
    }
    float cf[E];
    for (int v0 = 0; v0 < views; v0 += step) {
        const int nv = min(step, views - v0);
        if (v0 == 0 || per_view) {
            const float* src = a.sh + v0 * a.sh_view_stride + i * rf;
            if constexpr (staged) {
                rows_to_lds<E>(stage, a.sh + v0 * a.sh_view_stride + g0 * rf, rows_here);
#pragma unroll
                for (int e = 0; e < E; ++e) cf[e] = valid ? row_lds[e] : 0.0f;
            } else if (!valid) {
#pragma unroll
                for (int e = 0; e < E; ++e) cf[e] = 0.0f;
            } else if constexpr (vec) {
#pragma unroll
                for (int e = 0; e < E; e += 4) {
                    const float4 q = reinterpret_cast<const float4*>(src)[e >> 2];
                    cf[e] = q.x;
                    cf[e + 1] = q.y;
                    cf[e + 2] = q.z;
                    cf[e + 3] = q.w;
                }
            } else {
#pragma unroll
                for (int e = 0; e < E; ++e) cf[e] = src[e];
            }
        }
        // The group's directions and clamp-masked colour gradients.
        float unit[U][3], length[U], cg[U][3];
        bool vis[U];
        int radius_in[U];
        float up_in[U][3], centre_in[U][3];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int vc = min(v0 + u, views - 1);
            const int64_t row = (int64_t)vc * n + ic;
            radius_in[u] = a.radii[row];
#pragma unroll
            for (int c = 0; c < 3; ++c) up_in[u][c] = a.grad_colors[row * a.grad_colors_stride + c];
            if (DEG > 0) {
#pragma unroll
                for (int k = 0; k < 3; ++k) centre_in[u][k] = a.camera_centers[3 * vc + k];
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool use = valid && u < nv;
            const int radius = use ? radius_in[u] : 0;
            float up[3];
#pragma unroll
            for (int c = 0; c < 3; ++c) up[c] = use ? up_in[u][c] : 0.0f;
            vis[u] = radius > 0;
            length[u] = 1.0f;
#pragma unroll
            for (int k = 0; k < 3; ++k) unit[u][k] = 0.0f;
            if (DEG > 0 && use) {
                float dir[3];
#pragma unroll
                for (int k = 0; k < 3; ++k) dir[k] = mean[k] - centre_in[u][k];
                length[u] = length3(dir);
                const float l = sel_max(length[u], 1.0e-12f);
#pragma unroll
                for (int k = 0; k < 3; ++k) unit[u][k] = dir[k] / l;
            }
            // The forward colour before the clamp (sh_eval's order and rounding).
            float value[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int k = 0; k < KC; ++k) {
                const float b = sh_basis(unit[u], k);
#pragma unroll
                for (int c = 0; c < 3; ++c) value[c] = value[c] + b * cf[3 * k + c];
            }
#pragma unroll
            for (int c = 0; c < 3; ++c) cg[u][c] = (vis[u] && value[c] + 0.5f >= 0.0f) ? up[c] : 0.0f;
        }
        // Basis values are evaluated again below, not kept from the loop above.
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int k = 0; k < 3; ++k) unit[u][k] = opaque(unit[u][k]);
        float ug[U][3];
#pragma unroll
        for (int u = 0; u < U; ++u) ug[u][0] = ug[u][1] = ug[u][2] = 0.0f;
        float* dst = a.grad_sh ? a.grad_sh + (per_view ? v0 * a.sh_view_stride : 0) + i * rf : nullptr;
        const bool acc = !per_view && v0 > 0;
        float group[12];
        static_for<KC>([&](auto kk) {
#pragma clang fp contract(fast)
            constexpr int k = decltype(kk)::value;
            float g[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float b = sh_basis(unit[u], k);
#pragma unroll
                for (int c = 0; c < 3; ++c) g[c] += b * cg[u][c];
                if (DEG > 0) {
                    float bg[3];
                    sh_basis_grad(unit[u], k, bg);
                    const float d = cf[3 * k] * cg[u][0] + cf[3 * k + 1] * cg[u][1] + cf[3 * k + 2] * cg[u][2];
#pragma unroll
                    for (int q = 0; q < 3; ++q) ug[u][q] = ug[u][q] + d * bg[q];
                }
            }
            if constexpr (staged) {
                // The stage holds the wavefront's gradient rows until they are stored.
#pragma unroll
                for (int c = 0; c < 3; ++c) row_lds[3 * k + c] = acc ? row_lds[3 * k + c] + g[c] : g[c];
            } else {
                constexpr int slot = 3 * (k % 4);
#pragma unroll
                for (int c = 0; c < 3; ++c) group[slot + c] = g[c];
                if constexpr (k % 4 == 3 || k == KC - 1) {
                    if (dst && valid) put_sh_grads<vec, 3 * (k - k % 4), slot + 3>(dst, acc, group);
                }
            }
        });
        if constexpr (staged) {
            if (a.grad_sh && (per_view || v0 + step >= views))
                lds_to_rows<E>(stage, a.grad_sh + (per_view ? v0 * a.sh_view_stride : 0) + g0 * rf, rows_here);
        } else if (dst && valid && !acc) {
            for (int64_t e = E; e < rf; ++e) dst[e] = 0.0f;
        }
        // Direction gradients of the group's views.
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float gd[3] = {0.0f, 0.0f, 0.0f};
            if (DEG > 0 && vis[u]) {
#pragma clang fp contract(fast)
                const float il = __builtin_amdgcn_rcpf(sel_max(length[u], 1.0e-12f));  // gradient only
#pragma unroll
                for (int q = 0; q < 3; ++q) gd[q] = ug[u][q] * il;
                if (length[u] >= 1.0e-12f) {
                    const float f = (unit[u][0] * ug[u][0] + unit[u][1] * ug[u][1] + unit[u][2] * ug[u][2]) *
                                    __builtin_amdgcn_rcpf(length[u]);
#pragma unroll
                    for (int q = 0; q < 3; ++q) gd[q] = gd[q] - unit[u][q] * f;
                }
#pragma unroll
                for (int q = 0; q < 3; ++q) gm[q] += gd[q];
            }
            if constexpr (CAM) {
                const int v = v0 + u;
                if (u < nv && v < kMaxViewsCamLds) {
#pragma unroll
                    for (int q = 0; q < 3; ++q) {
                        const float sum = wave_sum_to_lane63(-gd[q]);
                        if (lane == 63) s_cam[wave][v][q] += sum;
                    }
                }
            }
        }
    }
    if (DEG > 0 && valid && a.grad_means) {
#pragma unroll
        for (int q = 0; q < 3; ++q) a.grad_means[3 * i + q] = gm_old[q] + gm[q];
    }
    if constexpr (CAM) {
        __syncthreads();
        for (int e = threadIdx.x; e < views * 3; e += kShRowBlock) {
            const int v = e / 3, k = e - v * 3;
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < kShRowBlock / 64; ++w) sum += s_cam[w][v][k];
            atomicAdd(a.grad_camera_centers + 3 * v + k, sum);
        }
    }
}

template <int DEG>
__global__ void sh_fwd_kernel(const float* __restrict__ coefficients, int rows, const float* __restrict__ dirs,
                              const int32_t* __restrict__ radii, int n, float* __restrict__ colors,
                              uint8_t* __restrict__ active) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    constexpr int KC = (DEG + 1) * (DEG + 1);
    float coef[3 * KC];
    for (int e = 0; e < 3 * KC; ++e) coef[e] = coefficients[i * rows * 3 + e];
    const float dir[3] = {dirs[3 * i], dirs[3 * i + 1], dirs[3 * i + 2]};
    const bool vis = radii ? radii[i] > 0 : true;
    float color[3], raw[3];
    sh_eval<DEG>(coef, dir, vis, color, raw);
    for (int k = 0; k < 3; ++k) {
        colors[3 * i + k] = color[k];
        if (active) active[3 * i + k] = (vis && raw[k] >= 0.0f) ? 1 : 0;
    }
}

template <int DEG>
__global__ void sh_bwd_kernel(const float* __restrict__ coefficients, int rows, const float* __restrict__ dirs,
                              const int32_t* __restrict__ radii, const uint8_t* __restrict__ active,
                              const float* __restrict__ upstream, int n, float* __restrict__ grad_coefficients,
                              float* __restrict__ grad_dirs) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    constexpr int KC = (DEG + 1) * (DEG + 1);
    float coef[3 * KC], gco[3 * KC], gd[3];
    for (int e = 0; e < 3 * KC; ++e) coef[e] = coefficients[i * rows * 3 + e];
    const float dir[3] = {dirs[3 * i], dirs[3 * i + 1], dirs[3 * i + 2]};
    const bool vis = radii ? radii[i] > 0 : true;
    const bool act[3] = {active[3 * i] != 0, active[3 * i + 1] != 0, active[3 * i + 2] != 0};
    const float up[3] = {upstream[3 * i], upstream[3 * i + 1], upstream[3 * i + 2]};
    sh_backward<DEG, false>(coef, dir, vis, act, up, gco, gd);
    if (grad_coefficients)
        for (int e = 0; e < rows * 3; ++e) grad_coefficients[i * rows * 3 + e] = e < 3 * KC ? gco[e] : 0.0f;
    if (grad_dirs)
        for (int k = 0; k < 3; ++k) grad_dirs[3 * i + k] = gd[k];
}

__global__ void metadata_kernel(const int32_t* __restrict__ radii, const float* __restrict__ centers,
                                const float* __restrict__ conics, int64_t n, float* __restrict__ means2d,
                                float* __restrict__ opacities, float* __restrict__ meta_conics) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const bool vis = radii[i] > 0;
    const float2 c = vis ? reinterpret_cast<const float2*>(centers)[i] : make_float2(0.0f, 0.0f);
    const float4 k = vis ? reinterpret_cast<const float4*>(conics)[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    reinterpret_cast<float2*>(means2d)[i] = c;
    opacities[i] = k.w;
    meta_conics[3 * i] = k.x;
    meta_conics[3 * i + 1] = k.y;
    meta_conics[3 * i + 2] = k.z;
}

// Row access of the SH kernels: float4 when rows start 16-byte aligned and
// the needed coefficients are whole float4s, scalar otherwise; with
// `allow_staged`, rows of exactly the needed coefficients are staged through
// LDS (coalesced copies).
inline int sh_row_mode(int deg, int sh_rows, const float* sh, int64_t view_stride, const float* grad_sh,
                       bool allow_staged) {
    const int e = 3 * (deg + 1) * (deg + 1);
    const bool aligned = (reinterpret_cast<uintptr_t>(sh) & 15) == 0 && (reinterpret_cast<uintptr_t>(grad_sh) & 15) == 0 &&
                         (view_stride & 3) == 0 && (sh_rows * 3) % 4 == 0 && e % 4 == 0;
    if (!aligned) return kRowsScalar;
    return allow_staged && sh_rows * 3 == e ? kRowsStaged : kRowsFloat4;
}

// Projection of every view, then (DEG >= 0) the colours in a second launch
// with one thread per Gaussian: the projection kernel then keeps its
// occupancy, and the SH basis is evaluated once per (Gaussian, view).
template <int DEG>
int launch_project_fwd(const gs3d_project_args& a, hipStream_t stream) {
    const dim3 grid(blocks_for(a.n, kProjBlock));
    if (a.means2d)
        hipLaunchKernelGGL((project_fwd_kernel<true>), grid, dim3(kProjBlock), 0, stream, a);
    else
        hipLaunchKernelGGL((project_fwd_kernel<false>), grid, dim3(kProjBlock), 0, stream, a);
    if constexpr (DEG >= 0) {
        const dim3 rgrid(blocks_for(a.n, kShRowBlock));
        if (sh_row_mode(DEG, a.sh_rows, a.sh, a.sh_view_stride, nullptr, false) == kRowsFloat4)
            hipLaunchKernelGGL((sh_rows_fwd_kernel<DEG, true>), rgrid, dim3(kShRowBlock), 0, stream, a);
        else
            hipLaunchKernelGGL((sh_rows_fwd_kernel<DEG, false>), rgrid, dim3(kShRowBlock), 0, stream, a);
    }
    return launch_status("gs3d_project_fwd");
}

inline dim3 persistent_grid(int64_t n) {
    int device = 0, cus = 256;
    if (hipGetDevice(&device) == hipSuccess) {
        int value = 0;
        if (hipDeviceGetAttribute(&value, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && value > 0)
            cus = value;
    }
    const int64_t needed = blocks_for(n, kProjBlock);
    const int64_t persistent = (int64_t)cus * 8;
    return dim3((unsigned)(needed < persistent ? needed : persistent));
}

// Projection VJP first (it writes grad_means), then the SH VJP (it adds the
// direction gradients to grad_means).
template <int DEG>
int launch_project_bwd(const gs3d_project_bwd_args& a, hipStream_t stream) {
    const dim3 grid = persistent_grid(a.n);
    if (a.grad_view || a.grad_projection)
        hipLaunchKernelGGL((project_bwd_kernel<true>), grid, dim3(kProjBlock), 0, stream, a);
    else
        hipLaunchKernelGGL((project_bwd_kernel<false>), grid, dim3(kProjBlock), 0, stream, a);
    if constexpr (DEG >= 0) {
        const int mode = sh_row_mode(DEG, a.sh_rows, a.sh, a.sh_view_stride, a.grad_sh, true);
        const dim3 rgrid(blocks_for(a.n, kShRowBlock));
        const bool cam = DEG > 0 && a.grad_camera_centers;
#define GS3D_SH_BWD_LAUNCH(M)                                                                              \
    do {                                                                                                   \
        if (cam)                                                                                           \
            hipLaunchKernelGGL((sh_rows_bwd_kernel<DEG, true, M>), rgrid, dim3(kShRowBlock), 0, stream, a);  \
        else                                                                                               \
            hipLaunchKernelGGL((sh_rows_bwd_kernel<DEG, false, M>), rgrid, dim3(kShRowBlock), 0, stream, a); \
    } while (0)
        if (mode == kRowsStaged)
            GS3D_SH_BWD_LAUNCH(kRowsStaged);
        else if (mode == kRowsFloat4)
            GS3D_SH_BWD_LAUNCH(kRowsFloat4);
        else
            GS3D_SH_BWD_LAUNCH(kRowsScalar);
#undef GS3D_SH_BWD_LAUNCH
    }
    return launch_status("gs3d_project_bwd");
}

}  // namespace gs3d

namespace gs3d {

// Tile counts of the SnugBox/AccuTile modes (gs3d/projection.py:150-161),
// over the projection's outputs: a separate pass keeps the tile traversal out
// of the projection kernel's registers.
__global__ void footprint_tiles_kernel(const float* __restrict__ centers, const float* __restrict__ conics,
                                       const int32_t* __restrict__ radii, int64_t rows, int gx, int gy, int mode,
                                       int32_t* __restrict__ tiles) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const int radius = radii[r];
    if (radius <= 0) return;
    tiles[r] = footprint_tiles(reinterpret_cast<const float2*>(centers)[r], reinterpret_cast<const float4*>(conics)[r],
                               radius, gx, gy, mode);
}

int project_fwd(const gs3d_project_args& a, hipStream_t s) {
    if (!a.sh) return launch_project_fwd<-1>(a, s);
    if (a.sh_degree < 0 || a.sh_degree > 3 || a.sh_rows < (a.sh_degree + 1) * (a.sh_degree + 1) || !a.colors ||
        (a.sh_degree > 0 && !a.camera_centers))
        return GS3D_ERR_ARGUMENT;
    switch (a.sh_degree) {
    case 0: return launch_project_fwd<0>(a, s);
    case 1: return launch_project_fwd<1>(a, s);
    case 2: return launch_project_fwd<2>(a, s);
    default: return launch_project_fwd<3>(a, s);
    }
}

}  // namespace gs3d

extern "C" int gs3d_project_fwd(const gs3d_project_args* args, void* stream) {
    if (!args) return GS3D_ERR_ARGUMENT;
    const gs3d_project_args& a = *args;
    if (a.n < 0 || a.views < 0 || a.width <= 0 || a.height <= 0) return GS3D_ERR_ARGUMENT;
    if (a.tile_mode < GS3D_TILE_RADIUS || a.tile_mode > GS3D_TILE_ACCUTILE) return GS3D_ERR_ARGUMENT;
    if (a.n == 0 || a.views == 0) return GS3D_OK;
    if (!a.means || !a.quats || !a.scales || !a.opacities || !a.view || !a.projection || !a.intrinsics ||
        !a.centers || !a.conics || !a.radii || !a.tiles || !a.depths)
        return GS3D_ERR_ARGUMENT;
    if ((reinterpret_cast<uintptr_t>(a.quats) & 15) || (reinterpret_cast<uintptr_t>(a.conics) & 15) ||
        (reinterpret_cast<uintptr_t>(a.centers) & 7) || (a.means2d && (reinterpret_cast<uintptr_t>(a.means2d) & 7)))
        return GS3D_ERR_ARGUMENT;
    if (a.means2d && (!a.meta_opacities || !a.meta_conics)) return GS3D_ERR_ARGUMENT;
    hipStream_t s = gs3d::as_stream(stream);
    const int status = gs3d::project_fwd(a, s);
    if (status != GS3D_OK || a.tile_mode == GS3D_TILE_RADIUS) return status;
    const int64_t rows = (int64_t)a.n * a.views;
    hipLaunchKernelGGL(gs3d::footprint_tiles_kernel, dim3(gs3d::blocks_for(rows, 256)), dim3(256), 0, s, a.centers,
                       a.conics, a.radii, rows, (a.width + 15) / 16, (a.height + 15) / 16, a.tile_mode, a.tiles);
    return gs3d::launch_status("gs3d_project_fwd");
}

extern "C" int gs3d_project_bwd(const gs3d_project_bwd_args* args, void* stream) {
    if (!args) return GS3D_ERR_ARGUMENT;
    const gs3d_project_bwd_args& a = *args;
    if (a.n < 0 || a.views < 0 || a.width <= 0 || a.height <= 0) return GS3D_ERR_ARGUMENT;
    if (a.n == 0 || a.views == 0) return GS3D_OK;
    if (!a.means || !a.quats || !a.scales || !a.opacities || !a.view || !a.projection || !a.intrinsics ||
        !a.radii || !a.grad_centers || !a.grad_conics || a.grad_centers_stride < 2 || a.grad_conics_stride < 4)
        return GS3D_ERR_ARGUMENT;
    if ((reinterpret_cast<uintptr_t>(a.quats) & 15) || (a.grad_quats && (reinterpret_cast<uintptr_t>(a.grad_quats) & 15)))
        return GS3D_ERR_ARGUMENT;
    const bool want_camera = a.grad_view || a.grad_projection || (a.sh && a.grad_camera_centers);
    if (want_camera && a.views > gs3d::kMaxViewsCamLds) return GS3D_ERR_UNSUPPORTED;
    hipStream_t s = gs3d::as_stream(stream);
    if (!a.sh) return gs3d::launch_project_bwd<-1>(a, s);
    if (a.sh_degree < 0 || a.sh_degree > 3 || a.sh_rows < (a.sh_degree + 1) * (a.sh_degree + 1) || !a.grad_colors ||
        a.grad_colors_stride < 3 || (a.sh_degree > 0 && !a.camera_centers))
        return GS3D_ERR_ARGUMENT;
    switch (a.sh_degree) {
    case 0: return gs3d::launch_project_bwd<0>(a, s);
    case 1: return gs3d::launch_project_bwd<1>(a, s);
    case 2: return gs3d::launch_project_bwd<2>(a, s);
    default: return gs3d::launch_project_bwd<3>(a, s);
    }
}

extern "C" int gs3d_sh_fwd(const float* coefficients, int32_t rows, const float* directions, const int32_t* radii,
                           int32_t n, int32_t degree, float* colors, uint8_t* active, void* stream) {
    if (n < 0 || degree < 0 || degree > 3 || rows < (degree + 1) * (degree + 1)) return GS3D_ERR_ARGUMENT;
    if (n == 0) return GS3D_OK;
    if (!coefficients || !directions || !colors) return GS3D_ERR_ARGUMENT;
    const dim3 grid(gs3d::blocks_for(n, 256)), block(256);
    hipStream_t s = gs3d::as_stream(stream);
    switch (degree) {
    case 0: hipLaunchKernelGGL(gs3d::sh_fwd_kernel<0>, grid, block, 0, s, coefficients, rows, directions, radii, n, colors, active); break;
    case 1: hipLaunchKernelGGL(gs3d::sh_fwd_kernel<1>, grid, block, 0, s, coefficients, rows, directions, radii, n, colors, active); break;
    case 2: hipLaunchKernelGGL(gs3d::sh_fwd_kernel<2>, grid, block, 0, s, coefficients, rows, directions, radii, n, colors, active); break;
    default: hipLaunchKernelGGL(gs3d::sh_fwd_kernel<3>, grid, block, 0, s, coefficients, rows, directions, radii, n, colors, active); break;
    }
    return gs3d::launch_status("gs3d_sh_fwd");
}

extern "C" int gs3d_sh_bwd(const float* coefficients, int32_t rows, const float* directions, const int32_t* radii,
                           const uint8_t* active, const float* upstream, int32_t n, int32_t degree,
                           float* grad_coefficients, float* grad_directions, void* stream) {
    if (n < 0 || degree < 0 || degree > 3 || rows < (degree + 1) * (degree + 1)) return GS3D_ERR_ARGUMENT;
    if (n == 0) return GS3D_OK;
    if (!coefficients || !directions || !active || !upstream) return GS3D_ERR_ARGUMENT;
    const dim3 grid(gs3d::blocks_for(n, 256)), block(256);
    hipStream_t s = gs3d::as_stream(stream);
    switch (degree) {
    case 0: hipLaunchKernelGGL(gs3d::sh_bwd_kernel<0>, grid, block, 0, s, coefficients, rows, directions, radii, active, upstream, n, grad_coefficients, grad_directions); break;
    case 1: hipLaunchKernelGGL(gs3d::sh_bwd_kernel<1>, grid, block, 0, s, coefficients, rows, directions, radii, active, upstream, n, grad_coefficients, grad_directions); break;
    case 2: hipLaunchKernelGGL(gs3d::sh_bwd_kernel<2>, grid, block, 0, s, coefficients, rows, directions, radii, active, upstream, n, grad_coefficients, grad_directions); break;
    default: hipLaunchKernelGGL(gs3d::sh_bwd_kernel<3>, grid, block, 0, s, coefficients, rows, directions, radii, active, upstream, n, grad_coefficients, grad_directions); break;
    }
    return gs3d::launch_status("gs3d_sh_bwd");
}

extern "C" int gs3d_metadata(const int32_t* radii, const float* centers, const float* conics, int64_t n,
                             float* means2d, float* opacities, float* meta_conics, void* stream) {
    if (n < 0) return GS3D_ERR_ARGUMENT;
    if (n == 0) return GS3D_OK;
    if (!radii || !centers || !conics || !means2d || !opacities || !meta_conics) return GS3D_ERR_ARGUMENT;
    hipLaunchKernelGGL(gs3d::metadata_kernel, dim3(gs3d::blocks_for(n, 256)), dim3(256), 0, gs3d::as_stream(stream),
                       radii, centers, conics, n, means2d, opacities, meta_conics);
    return gs3d::launch_status("gs3d_metadata");
}
