// gs3d_oracle.cpp — CPU restatement of the original-3DGS (gs3d) path of
// YukiNagato/dsl_splat, used ONLY to test the HIP kernels' results.
//
// TEST INFRASTRUCTURE.  Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg load this library.  The product (dsl_splat_amd) never
// links, imports or calls it.
//
// Every function follows the reference kernel it names, operation by
// operation, in float32 with contraction off (built with -ffp-contract=off);
// fmaf appears exactly where the reference calls fused_multiply_add / fmaf.
// The projection forward and its VJP are templates so that a float64
// instantiation can be checked against finite differences.
//
// Choices the reference leaves to the CUDA compiler (Warp's default fuse_fp in
// project/duplicate/render) are fixed here and documented at each site:
//   * projection scalar arithmetic: no contraction;
//   * blending: the power/colour contractions in blend_power()/blend_accum();
//   * exp: gs_expf() below, a fixed-sequence Cody-Waite + Taylor routine.
// The HIP kernels implement the same choices, so integer outputs and the
// forward image are bit-exact between the two; reductions whose order the
// GPU does not fix (atomics) are compared with a tolerance.
//
// Parity pins (tests/test_oracle_*.py): closed forms for camera rows,
// projection special cases, SH0 and the blend of a single Gaussian; a NumPy
// brute-force renderer; numpy.lexsort / searchsorted for scan, keys, sort and
// ranges; float64 central differences for the projection, SH and blend VJPs;
// known-answer checks of the three custom adjoints.

#include <algorithm>
#include <cmath>
#include <limits>
#include <cstdint>
#include <cstring>
#include <numeric>
#include <vector>

#include <omp.h>
#include <parallel/algorithm>

#include "gs3d_hip.h"

namespace {

// ---------------------------------------------------------------------------
// exp used by blending (gs3d/render.py:96, :287 call wp.exp).  Fixed sequence:
// x = k*ln2 + r with k = rint(x*log2 e), r by two-constant Cody-Waite
// reduction (ln2_hi has 15 significant bits so k*ln2_hi is exact), then the
// degree-7 Taylor polynomial of exp(r) on |r| <= ln2/2 in Horner form, scaled
// by 2^k.  Below -86 the result is flushed to 0 (it is < 2^-124, far below the
// 1/255 blending threshold and keeps every intermediate normal).
// ---------------------------------------------------------------------------
inline float gs_expf(float x) {
    if (x < -86.0f) return 0.0f;
    const float k = rintf(x * 1.44269502e+00f);
    float r = fmaf(k, -6.93145752e-01f, x);
    r = fmaf(k, -1.42860677e-06f, r);
    float p = 1.98412701e-04f;            // 1/5040
    p = fmaf(p, r, 1.38888892e-03f);      // 1/720
    p = fmaf(p, r, 8.33333377e-03f);      // 1/120
    p = fmaf(p, r, 4.16666679e-02f);      // 1/24
    p = fmaf(p, r, 1.66666672e-01f);      // 1/6
    p = fmaf(p, r, 5.00000000e-01f);      // 1/2
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)k);
}

// ---------------------------------------------------------------------------
// Natural log of the alpha level used by the SnugBox/AccuTile footprint
// (splatting/intersections.py:68 calls wp.log).  Fixed sequence of IEEE
// double operations, rounded to float once: x = m * 2^e with m in
// [sqrt(1/2), sqrt(2)), ln m = 2 atanh(s), s = (m - 1)/(m + 1), |s| <= 0.1716,
// atanh by its Taylor series through s^23 (truncation below 1e-19).
// ---------------------------------------------------------------------------
inline float gs_logf(float x) {
    if (std::isnan(x) || x < 0.0f) return std::numeric_limits<float>::quiet_NaN();
    if (x == 0.0f) return -std::numeric_limits<float>::infinity();
    if (std::isinf(x)) return x;
    int e = 0;
    if (x < 1.17549435e-38f) {  // subnormal: scale into the normal range
        x *= 18446744073709551616.0f;  // 2^64
        e = -64;
    }
    uint32_t bits;
    std::memcpy(&bits, &x, 4);
    e += (int)(bits >> 23) - 127;
    bits = (bits & 0x007FFFFFu) | 0x3F800000u;  // mantissa in [1, 2)
    float mf;
    std::memcpy(&mf, &bits, 4);
    double m = (double)mf;
    if (m > 1.4142135623730951) {
        m = m * 0.5;
        e += 1;
    }
    const double s = (m - 1.0) / (m + 1.0);
    const double s2 = s * s;
    double p = 1.0 / 23.0;
    p = p * s2 + 1.0 / 21.0;
    p = p * s2 + 1.0 / 19.0;
    p = p * s2 + 1.0 / 17.0;
    p = p * s2 + 1.0 / 15.0;
    p = p * s2 + 1.0 / 13.0;
    p = p * s2 + 1.0 / 11.0;
    p = p * s2 + 1.0 / 9.0;
    p = p * s2 + 1.0 / 7.0;
    p = p * s2 + 1.0 / 5.0;
    p = p * s2 + 1.0 / 3.0;
    p = p * s2 + 1.0;
    return (float)(2.0 * s * p + (double)e * 0.6931471805599453);
}

// ---------------------------------------------------------------------------
// Quaternion normalisation the reference applies before projection
// (inputs.py:252, torch.nn.functional.normalize): q / max(|q|, 1e-12), and
// its VJP g -> (g - u (u.g)) / |q| (g / 1e-12 where the norm is clamped).
// ---------------------------------------------------------------------------
inline float normalize_quat(const float* q, float* u) {
    const float norm = sqrtf(((q[0] * q[0] + q[1] * q[1]) + q[2] * q[2]) + q[3] * q[3]);
    const float d = norm < 1e-12f ? 1e-12f : norm;
    for (int k = 0; k < 4; ++k) u[k] = q[k] / d;
    return norm;
}

template <class T> inline void normalize_quat_vjp(const float* u, float norm, T* g) {
    if (norm > 1e-12f) {
        const T dot = ((T(u[0]) * g[0] + T(u[1]) * g[1]) + T(u[2]) * g[2]) + T(u[3]) * g[3];
        for (int k = 0; k < 4; ++k) g[k] = (g[k] - T(u[k]) * dot) / T(norm);
    } else {
        for (int k = 0; k < 4; ++k) g[k] = g[k] / T(1e-12f);
    }
}

// ---------------------------------------------------------------------------
// Small fixed-size math in a scalar template T (float for the oracle,
// double for finite-difference checks).
// ---------------------------------------------------------------------------
template <class T> inline T fma_(T a, T b, T c) { return std::fma(a, b, c); }
template <> inline float fma_<float>(float a, float b, float c) { return fmaf(a, b, c); }

// ---------------------------------------------------------------------------
// Running error analysis (Wilkinson) of the gradient path, used to state how
// far two float32 evaluations of the same gradient in different operation
// orders may lie apart.  Err carries the value v exactly as the float32
// oracle computes it (every branch, clamp and threshold therefore decides
// identically) and two first-order bounds in double on |v - exact|:
//   p -- the part inherited from errors in the inputs (e.g. the upstream
//        gradients of a VJP, which arrive with their own bound),
//   r -- the part caused by this computation's own roundings.
// Each operation propagates both (|y| e_x + |x| e_y for a product,
// (e_x + |q| e_y) / |y| for a quotient, sums for sums and differences) and
// adds u |result| to r for its own rounding, u = 2^-24.
// ---------------------------------------------------------------------------
constexpr double kUnitRoundoff = 1.0 / 16777216.0;

struct Err {
    float v;
    double p, r;
    Err() = default;
    Err(float x) : v(x), p(0.0), r(0.0) {}
    Err(double x) : v((float)x), p(0.0), r(0.0) {}
    Err(int x) : v((float)x), p(0.0), r(0.0) {}
    Err(float x, double prop, double round) : v(x), p(prop), r(round) {}
};
inline double ad(float x) { return std::fabs((double)x); }
inline Err operator+(Err a, Err b) {
    const float v = a.v + b.v;
    return Err(v, a.p + b.p, a.r + b.r + kUnitRoundoff * ad(v));
}
inline Err operator-(Err a, Err b) {
    const float v = a.v - b.v;
    return Err(v, a.p + b.p, a.r + b.r + kUnitRoundoff * ad(v));
}
inline Err operator-(Err a) { return Err(-a.v, a.p, a.r); }
inline Err operator*(Err a, Err b) {
    const float v = a.v * b.v;
    return Err(v, ad(b.v) * a.p + ad(a.v) * b.p, ad(b.v) * a.r + ad(a.v) * b.r + kUnitRoundoff * ad(v));
}
inline Err operator/(Err a, Err b) {
    const float v = a.v / b.v;
    const double d = ad(b.v);
    return Err(v, (a.p + ad(v) * b.p) / d, (a.r + ad(v) * b.r) / d + kUnitRoundoff * ad(v));
}
inline Err& operator+=(Err& a, Err b) { return a = a + b; }
inline Err& operator-=(Err& a, Err b) { return a = a - b; }
inline Err& operator*=(Err& a, Err b) { return a = a * b; }
inline bool operator<(Err a, Err b) { return a.v < b.v; }
inline bool operator>(Err a, Err b) { return a.v > b.v; }
inline bool operator<=(Err a, Err b) { return a.v <= b.v; }
inline bool operator>=(Err a, Err b) { return a.v >= b.v; }
inline bool operator==(Err a, Err b) { return a.v == b.v; }
inline bool operator!=(Err a, Err b) { return a.v != b.v; }
template <> inline Err fma_<Err>(Err a, Err b, Err c) {
    const float v = fmaf(a.v, b.v, c.v);
    return Err(v, ad(b.v) * a.p + ad(a.v) * b.p + c.p, ad(b.v) * a.r + ad(a.v) * b.r + c.r + kUnitRoundoff * ad(v));
}
inline float val(float x) { return x; }
inline float val(Err x) { return x.v; }

template <class T> struct M3 { T m[3][3]; };
template <class T> struct M4 { T m[4][4]; };

template <class T> M3<T> transpose(const M3<T>& a) {
    M3<T> r;
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j) r.m[i][j] = a.m[j][i];
    return r;
}

// splatting/math.py:31-41 reference_matmul: fma(a[r,2], b[2,c],
// fma(a[r,0], b[0,c], a[r,1]*b[1,c])).
template <class T> M3<T> ref_matmul(const M3<T>& a, const M3<T>& b) {
    M3<T> r;
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j)
            r.m[i][j] = fma_(a.m[i][2], b.m[2][j], fma_(a.m[i][0], b.m[0][j], a.m[i][1] * b.m[1][j]));
    return r;
}

// splatting/math.py:44-47 point_row: fma(M[r,2], z, fma(M[r,0], x, M[r,1]*y)) + M[r,3].
template <class T> T point_row(const M4<T>& m, int r, const T p[3]) {
    T xy = fma_(m.m[r][0], p[0], m.m[r][1] * p[1]);
    return fma_(m.m[r][2], p[2], xy) + m.m[r][3];
}

// primitives/math.py:33-45 glm_rotation (rounded products where __fmul_rn /
// __fadd_rn / __fsub_rn are used, fmaf elsewhere).
template <class T> M3<T> glm_rotation(const T q[4]) {
    const T r = q[0], x = q[1], y = q[2], z = q[3];
    const T yy = y * y, zz = z * z;
    const T rz = r * z, xz = x * z, rx = r * x;
    const T d0 = yy + zz, d1 = fma_(x, x, zz), d2 = fma_(x, x, yy);
    M3<T> R;
    R.m[0][0] = T(1) - (d0 + d0);
    R.m[0][1] = T(2) * fma_(x, y, rz);
    R.m[0][2] = T(2) * fma_(-r, y, xz);
    R.m[1][0] = T(2) * fma_(x, y, -rz);
    R.m[1][1] = T(1) - (d1 + d1);
    R.m[1][2] = T(2) * fma_(y, z, rx);
    R.m[2][0] = T(2) * fma_(r, y, xz);
    R.m[2][1] = T(2) * fma_(y, z, -rx);
    R.m[2][2] = T(1) - (d2 + d2);
    return R;
}

template <class T> T clampv(T v, T lo, T hi) { return std::min(std::max(v, lo), hi); }

template <class T> M4<T> load44(const float* p) {
    M4<T> m;
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j) m.m[i][j] = T(p[4 * i + j]);
    return m;
}

// ---------------------------------------------------------------------------
// Projection forward, gs3d/projection.py:37-86 (screen_covariance) and
// splatting/geometry.py:22-123.
// ---------------------------------------------------------------------------
template <class T> struct CovState {
    // Intermediates kept for the VJP.
    T t[3];          // clamped camera point (geometry.py:33-39)
    T pos[3];        // unclamped camera point
    M3<T> R, M, Sigma, J, W, Tm, X, cov2;
    T limx, limy;
};

template <class T>
void screen_covariance(const T pos[3], const T q[4], const T s[3], const M4<T>& V,
                       int width, int height, T fx, T fy, CovState<T>& st, T cov[3]) {
    // projection.py:48-52 limits, clamp_point geometry.py:33-39.
    const T limx = T(1.3) * T(width) / (T(2) * fx);
    const T limy = T(1.3) * T(height) / (T(2) * fy);
    st.limx = limx;
    st.limy = limy;
    for (int i = 0; i < 3; ++i) st.pos[i] = pos[i];
    st.t[0] = clampv(pos[0] / pos[2], -limx, limx) * pos[2];
    st.t[1] = clampv(pos[1] / pos[2], -limy, limy) * pos[2];
    st.t[2] = pos[2];
    st.R = glm_rotation(q);
    M3<T> S{};
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j) S.m[i][j] = T(0);
    S.m[0][0] = s[0];
    S.m[1][1] = s[1];
    S.m[2][2] = s[2];
    st.M = ref_matmul(S, st.R);
    st.Sigma = ref_matmul(transpose(st.M), st.M);
    const T* t = st.t;
    M3<T> J{};
    J.m[0][0] = fx / t[2]; J.m[0][1] = T(0); J.m[0][2] = T(0);
    J.m[1][0] = T(0); J.m[1][1] = fy / t[2]; J.m[1][2] = T(0);
    J.m[2][0] = -(fx * t[0]) / (t[2] * t[2]);
    J.m[2][1] = -(fy * t[1]) / (t[2] * t[2]);
    J.m[2][2] = T(0);
    st.J = J;
    M3<T> W;
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j) W.m[i][j] = V.m[j][i];
    st.W = W;
    st.Tm = ref_matmul(W, J);
    st.X = ref_matmul(transpose(st.Tm), transpose(st.Sigma));
    st.cov2 = ref_matmul(st.X, st.Tm);
    cov[0] = st.cov2.m[0][0] + T(0.3);
    cov[1] = st.cov2.m[1][0];
    cov[2] = st.cov2.m[1][1] + T(0.3);
}

// splatting/geometry.py:54-58 invert_covariance.
template <class T> void invert_covariance(const T cov[3], T out[3]) {
    const T a = cov[0], b = cov[1], c = cov[2];
    const T inv = T(1) / (a * c - b * b);
    out[0] = c * inv;
    out[1] = -b * inv;
    out[2] = a * inv;
}

// splatting/geometry.py:106-123 pixel_center: fp32 perspective divide, fp64
// viewport transform, rounded once to fp32.
template <class T> void pixel_center(const T mean[3], const M4<T>& P, int width, int height,
                                     T out[2], T clip[4], T* inv_w_out) {
    for (int r = 0; r < 4; ++r) clip[r] = point_row(P, r, mean);
    const T inv_w = T(1) / (clip[3] + T(0.0000001));
    *inv_w_out = inv_w;
    const double ndc_x = double(clip[0] * inv_w);
    const double ndc_y = double(clip[1] * inv_w);
    out[0] = T(((ndc_x + 1.0) * double(width) - 1.0) * 0.5);
    out[1] = T(((ndc_y + 1.0) * double(height) - 1.0) * 0.5);
}

// splatting/geometry.py:22-30 tile_bounds (CUDA getRect truncation).
inline void tile_bounds(const float c[2], int radius, int gx, int gy, int b[4]) {
    auto trunc_clamp = [](float v, int hi) {
        int i = (int)v;
        return std::min(std::max(i, 0), hi);
    };
    const float r = (float)radius;
    b[0] = trunc_clamp((c[0] - r) / 16.0f, gx);
    b[1] = trunc_clamp((c[1] - r) / 16.0f, gy);
    b[2] = trunc_clamp(((c[0] + r) + 16.0f - 1.0f) / 16.0f, gx);
    b[3] = trunc_clamp(((c[1] + r) + 16.0f - 1.0f) / 16.0f, gy);
}

// ---------------------------------------------------------------------------
// SnugBox / AccuTile intersections, splatting/intersections.py:46-218,
// restated step by step (float32 unless the reference converts).
// ---------------------------------------------------------------------------
struct Ellipse {
    float center[2] = {0.0f, 0.0f};
    float conic[3] = {0.0f, 0.0f, 0.0f};
    float level = 0.0f, determinant = 0.0f;
    float extent[2] = {0.0f, 0.0f};
    int bounds[4] = {0, 0, 0, 0};
    bool precise = false;
};

inline float clampf(float x, float lo, float hi) { return std::min(std::max(x, lo), hi); }

// intersections.py:46-116 footprint.
Ellipse footprint(const float center[2], const float conic[4], int radius, int gx, int gy) {
    Ellipse r;
    r.center[0] = center[0];
    r.center[1] = center[1];
    r.conic[0] = conic[0];
    r.conic[1] = conic[1];
    r.conic[2] = conic[2];
    tile_bounds(center, radius, gx, gy, r.bounds);
    const float a = conic[0], b = conic[1], c = conic[2];
    const float det = (float)((double)a * (double)c - (double)b * (double)b);
    if (conic[3] < 1.0f / 255.0f) {
        r.bounds[0] = r.bounds[1] = r.bounds[2] = r.bounds[3] = 0;
        return r;
    }
    if (!(a > 0.0f && c > 0.0f && det > 0.0f)) return r;
    const float level = 2.0f * gs_logf(conic[3] * 255.0f);
    const float reach = (float)radius + 32.0f;
    const float roundoff = 9.5367431640625e-07f * ((a + 2.0f * std::fabs(b) + c) * reach * reach + std::fabs(level) + 1.0f);
    r.level = std::max(0.0f, level) + roundoff;
    r.determinant = det;
    r.extent[0] = sqrtf(r.level * c / det);
    r.extent[1] = sqrtf(r.level * a / det);
    if (!(std::isfinite(r.extent[0]) && std::isfinite(r.extent[1]))) return r;
    const int lo_x = (int)clampf(floorf((center[0] - r.extent[0]) / 16.0f), 0.0f, (float)gx);
    const int lo_y = (int)clampf(floorf((center[1] - r.extent[1]) / 16.0f), 0.0f, (float)gy);
    const int hi_x = (int)clampf(floorf((center[0] + r.extent[0]) / 16.0f) + 1.0f, 0.0f, (float)gx);
    const int hi_y = (int)clampf(floorf((center[1] + r.extent[1]) / 16.0f) + 1.0f, 0.0f, (float)gy);
    r.bounds[0] = std::max(r.bounds[0], lo_x);
    r.bounds[1] = std::max(r.bounds[1], lo_y);
    r.bounds[2] = std::min(r.bounds[2], hi_x);
    r.bounds[3] = std::min(r.bounds[3], hi_y);
    r.precise = true;
    return r;
}

// intersections.py:119-130: where the line u = 16*line meets the ellipse.
void line_intersection(const Ellipse& e, int line, bool is_y, float out[2]) {
    float u = e.center[0], v = e.center[1];
    const float b = e.conic[1];
    float c = e.conic[2], extent_u = e.extent[0];
    if (is_y) {
        std::swap(u, v);
        c = e.conic[0];
        extent_u = e.extent[1];
    }
    const float h = clampf((float)(line * 16) - u, -extent_u, extent_u);
    const float root = sqrtf(std::max(0.0f, e.level * c - e.determinant * h * h));
    out[0] = v + (-b * h - root) / c;
    out[1] = v + (-b * h + root) / c;
}

// intersections.py:133-157: tile span of strip `row`.
void strip_span(const Ellipse& e, int row, bool is_y, const float low[2], const float high[2], int out[2]) {
    float u = e.center[0], v = e.center[1];
    float a = e.conic[0];
    const float b = e.conic[1];
    float extent = e.extent[1];
    int lower = e.bounds[1], upper = e.bounds[3];
    if (is_y) {
        std::swap(u, v);
        a = e.conic[2];
        extent = e.extent[0];
        lower = e.bounds[0];
        upper = e.bounds[2];
    }
    float lo = std::min(low[0], high[0]), hi = std::max(low[1], high[1]);
    const float arg_min = b * extent / a, arg_max = -b * extent / a;
    const float h0 = (float)(row * 16) - u, h1 = (float)((row + 1) * 16) - u;
    if (h0 <= arg_min && arg_min <= h1) lo = v - extent;
    if (h0 <= arg_max && arg_max <= h1) hi = v + extent;
    out[0] = (int)clampf(floorf(lo / 16.0f), (float)lower, (float)upper);
    out[1] = (int)clampf(floorf(hi / 16.0f) + 1.0f, (float)lower, (float)upper);
}

// intersections.py:160-218 visit: the tiles of one projected Gaussian in the
// reference's traversal order; returns the count and, when `tiles` is
// non-null, writes the tile indices (row-major within the view).
int visit_tiles(int mode, const float center[2], const float conic[4], int radius, int gx, int gy,
                int64_t* tiles) {
    Ellipse e;
    tile_bounds(center, radius, gx, gy, e.bounds);
    if (mode != GS3D_TILE_RADIUS) e = footprint(center, conic, radius, gx, gy);
    const int* bounds = e.bounds;
    const int nx = std::max(0, bounds[2] - bounds[0]), ny = std::max(0, bounds[3] - bounds[1]);
    if (nx == 0 || ny == 0) return 0;
    bool is_y = true;
    if (mode == GS3D_TILE_ACCUTILE) is_y = ny < nx;
    int start = bounds[1], end = bounds[3];
    if (!is_y) {
        start = bounds[0];
        end = bounds[2];
    }
    if (mode != GS3D_TILE_ACCUTILE && !tiles) return nx * ny;
    float low[2] = {0.0f, 0.0f}, high[2];
    if (mode == GS3D_TILE_ACCUTILE && e.precise) line_intersection(e, start, is_y, low);
    int count = 0;
    for (int row = start; row < end; ++row) {
        int span[2] = {bounds[0], bounds[2]};
        if (!is_y) {
            span[0] = bounds[1];
            span[1] = bounds[3];
        }
        if (mode == GS3D_TILE_ACCUTILE && e.precise) {
            line_intersection(e, row + 1, is_y, high);
            strip_span(e, row, is_y, low, high, span);
            low[0] = high[0];
            low[1] = high[1];
        }
        if (tiles)
            for (int col = span[0]; col < span[1]; ++col)
                tiles[count + col - span[0]] = is_y ? (int64_t)row * gx + col : (int64_t)col * gx + row;
        count += std::max(0, span[1] - span[0]);
    }
    return count;
}

// gs3d/projection.py:89-164 project, one Gaussian in one view.
struct ProjOut {
    float center[2], conic[4];
    int radius, tiles;
    float depth;
};

bool project_one(const float* mean, const float* quat, const float* scale, float opacity,
                 const float* view, const float* proj, const float* K, int width, int height,
                 float near_plane, float far_plane, float radius_clip, ProjOut& o, int tile_mode = GS3D_TILE_RADIUS) {
    o = ProjOut{};
    const M4<float> V = load44<float>(view);
    float t4[4];
    for (int r = 0; r < 4; ++r) t4[r] = point_row(V, r, mean);
    if (t4[2] <= near_plane || t4[2] >= far_plane) return false;
    CovState<float> st;
    float cov[3];
    screen_covariance<float>(t4, quat, scale, V, width, height, K[0], K[4], st, cov);
    const float a = cov[0], b = cov[1], c = cov[2];
    const float det = a * c - b * b;
    if (det == 0.0f) return false;
    const float mid = 0.5f * (a + c);
    const int radius = (int)ceilf(3.0f * sqrtf(mid + sqrtf(std::max(0.1f, mid * mid - det))));
    if ((float)radius <= radius_clip) return false;
    float center[2], clip[4], inv_w;
    pixel_center<float>(mean, load44<float>(proj), width, height, center, clip, &inv_w);
    int bnd[4];
    tile_bounds(center, radius, (width + 15) / 16, (height + 15) / 16, bnd);
    const int count = (bnd[2] - bnd[0]) * (bnd[3] - bnd[1]);
    if (count == 0) return false;
    float inv[3];
    invert_covariance<float>(cov, inv);
    o.center[0] = center[0];
    o.center[1] = center[1];
    o.conic[0] = inv[0];
    o.conic[1] = inv[1];
    o.conic[2] = inv[2];
    o.conic[3] = opacity;
    o.radius = radius;
    o.tiles = count;
    if (tile_mode != GS3D_TILE_RADIUS)  // projection.py:150-161
        o.tiles = visit_tiles(tile_mode, o.center, o.conic, radius, (width + 15) / 16, (height + 15) / 16, nullptr);
    o.depth = t4[2];
    return true;
}

// ---------------------------------------------------------------------------
// SH, primitives/sh.py:7-79 (basis, evaluate).  Constants are the float32
// roundings of the reference literals; products evaluate left to right.
// ---------------------------------------------------------------------------
inline float sh_basis(const float u[3], int k) {
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

// Gradient of sh_basis w.r.t. the unit direction (what wp.grad(basis)
// returns at primitives/sh.py:127), derived from the polynomials above.
inline void sh_basis_grad(const float u[3], int k, float g[3]) {
    const float x = u[0], y = u[1], z = u[2];
    g[0] = g[1] = g[2] = 0.0f;
    const float C1 = 0.4886025119029199f, C4 = 1.0925484305920792f, C6 = 0.31539156525252005f,
                C8 = 0.5462742152960396f, C9 = 0.5900435899266435f, C10 = 2.890611442640554f,
                C11 = 0.4570457994644658f, C12 = 0.3731763325901154f, C14 = 1.445305721320277f;
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
    case 9:  // -C9 * y * (3x^2 - y^2) = -C9 (3x^2 y - y^3)
        g[0] = -C9 * (6.0f * x * y);
        g[1] = -C9 * (3.0f * x * x - 3.0f * y * y);
        break;
    case 10: g[0] = C10 * y * z; g[1] = C10 * x * z; g[2] = C10 * x * y; break;
    case 11:  // -C11 * y * (4z^2 - x^2 - y^2)
        g[0] = -C11 * (-2.0f * x * y);
        g[1] = -C11 * (4.0f * z * z - x * x - 3.0f * y * y);
        g[2] = -C11 * (8.0f * y * z);
        break;
    case 12:  // C12 * z * (2z^2 - 3x^2 - 3y^2)
        g[0] = C12 * (-6.0f * x * z);
        g[1] = C12 * (-6.0f * y * z);
        g[2] = C12 * (6.0f * z * z - 3.0f * x * x - 3.0f * y * y);
        break;
    case 13:  // -C11 * x * (4z^2 - x^2 - y^2)
        g[0] = -C11 * (4.0f * z * z - 3.0f * x * x - y * y);
        g[1] = -C11 * (-2.0f * x * y);
        g[2] = -C11 * (8.0f * x * z);
        break;
    case 14:  // C14 * z * (x^2 - y^2)
        g[0] = C14 * (2.0f * x * z);
        g[1] = C14 * (-2.0f * y * z);
        g[2] = C14 * (x * x - y * y);
        break;
    default:  // -C9 * x * (x^2 - 3y^2)
        g[0] = -C9 * (3.0f * x * x - 3.0f * y * y);
        g[1] = -C9 * (-6.0f * x * y);
        break;
    }
}

// wp.length (dot without contraction, then sqrt) and the guarded divide of
// primitives/sh.py:67, :113-114.
inline float length3(const float d[3]) { return sqrtf(d[0] * d[0] + d[1] * d[1] + d[2] * d[2]); }

// primitives/sh.py:58-77 for one row: returns the pre-clamp value in raw.
inline void sh_eval(const float* coef, const float dir[3], int degree, bool visible,
                    float color[3], float raw[3]) {
    float value[3] = {0.0f, 0.0f, 0.0f};
    if (visible) {
        float unit[3] = {0.0f, 0.0f, 0.0f};
        if (degree > 0) {
            const float len = std::max(length3(dir), 1.0e-12f);
            for (int i = 0; i < 3; ++i) unit[i] = dir[i] / len;
        }
        const int count = (degree + 1) * (degree + 1);
        for (int k = 0; k < count; ++k) {
            const float b = sh_basis(unit, k);
            for (int ch = 0; ch < 3; ++ch) value[ch] = value[ch] + b * coef[3 * k + ch];
        }
        for (int ch = 0; ch < 3; ++ch) value[ch] = value[ch] + 0.5f;
    }
    for (int ch = 0; ch < 3; ++ch) {
        raw[ch] = value[ch];
        color[ch] = std::max(value[ch], 0.0f);
    }
}

// primitives/sh.py:100-136 for one row.  active[ch] is the saved clamp mask.
// T is float (the oracle) or Err (its running error analysis); the
// direction, basis values and basis gradients are forward quantities.
template <class T>
inline void sh_backward_row(const float* coef, const float dir[3], int degree, bool visible,
                            const bool active[3], const T upstream[3], T* grad_coef,
                            int rows, T grad_dir[3]) {
    grad_dir[0] = grad_dir[1] = grad_dir[2] = T(0.0f);
    if (grad_coef)
        for (int i = 0; i < rows * 3; ++i) grad_coef[i] = T(0.0f);
    if (!visible) return;
    T cg[3];
    for (int ch = 0; ch < 3; ++ch) cg[ch] = active[ch] ? upstream[ch] : T(0.0f);
    float unit[3] = {0.0f, 0.0f, 0.0f}, length = 1.0f;
    if (degree > 0) {
        length = length3(dir);
        const float l = std::max(length, 1.0e-12f);
        for (int i = 0; i < 3; ++i) unit[i] = dir[i] / l;
    }
    T ug[3] = {T(0.0f), T(0.0f), T(0.0f)};
    const int count = (degree + 1) * (degree + 1);
    for (int k = 0; k < count; ++k) {
        const float b = sh_basis(unit, k);
        if (grad_coef)
            for (int ch = 0; ch < 3; ++ch) grad_coef[3 * k + ch] = T(b) * cg[ch];
        float bg[3];
        sh_basis_grad(unit, k, bg);
        const T d = T(coef[3 * k]) * cg[0] + T(coef[3 * k + 1]) * cg[1] + T(coef[3 * k + 2]) * cg[2];
        for (int i = 0; i < 3; ++i) ug[i] = ug[i] + d * T(bg[i]);
    }
    if (degree > 0) {
        const float l = std::max(length, 1.0e-12f);
        for (int i = 0; i < 3; ++i) grad_dir[i] = ug[i] / T(l);
        if (length >= 1.0e-12f) {
            const T dot = T(unit[0]) * ug[0] + T(unit[1]) * ug[1] + T(unit[2]) * ug[2];
            const T f = dot / T(length);
            for (int i = 0; i < 3; ++i) grad_dir[i] = grad_dir[i] - T(unit[i]) * f;
        }
    }
}

// ---------------------------------------------------------------------------
// Projection VJP: the reverse pass of gs3d/projection.py:198-210
// (projection_loss) as wp.grad evaluates it, with the custom adjoints of
// splatting/geometry.py:42-51 (clamp), :61-71 (inverse covariance) and
// splatting/math.py:13-28 (rotation); fmaf adjoint of primitives/math.py:16.
// ---------------------------------------------------------------------------
template <class T> struct ProjGrad {
    T mean[3], quat[4], scale[3], opacity;
    T view[4][4], proj[4][4];
};

// dC = A*B; given gC, accumulate gA += gC*B^T, gB += A^T*gC.
template <class T> void matmul_vjp(const M3<T>& A, const M3<T>& B, const M3<T>& gC, M3<T>& gA, M3<T>& gB) {
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j) {
            T sa = T(0), sb = T(0);
            for (int k = 0; k < 3; ++k) {
                sa += gC.m[i][k] * B.m[j][k];
                sb += A.m[k][i] * gC.m[k][j];
            }
            gA.m[i][j] += sa;
            gB.m[i][j] += sb;
        }
}

template <class T> M3<T> zero3() {
    M3<T> z;
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j) z.m[i][j] = T(0);
    return z;
}

template <class T>
void projection_vjp(const T mean[3], const T q[4], const T s[3], T opacity, const M4<T>& V,
                    const M4<T>& P, int width, int height, T fx, T fy, const T gc[2],
                    const T gk[4], ProjGrad<T>& g) {
    std::memset(&g, 0, sizeof(g));
    // Forward recomputation.
    T pos[3];
    for (int r = 0; r < 3; ++r) pos[r] = point_row(V, r, mean);
    CovState<T> st;
    T cov[3];
    screen_covariance<T>(pos, q, s, V, width, height, fx, fy, st, cov);
    // conic = invert_covariance(cov) + opacity.
    g.opacity = gk[3];
    {
        // splatting/geometry.py:61-71 adj_invert_covariance.
        const T a = cov[0], b = cov[1], c = cov[2];
        const T det = a * c - b * b;
        const T factor = T(1) / (det * det + T(0.0000001));
        const T x = gk[0], y = gk[1], z = gk[2];
        const T ga = factor * (-c * c * x + b * c * y + (det - a * c) * z);
        const T gb = factor * (T(2) * b * c * x - (det + T(2) * b * b) * y + T(2) * a * b * z);
        const T gcv = factor * (-a * a * z + a * b * y + (det - a * c) * x);
        // cov = (cov2[0,0]+0.3, cov2[1,0], cov2[1,1]+0.3)
        M3<T> gcov2 = zero3<T>();
        gcov2.m[0][0] = ga;
        gcov2.m[1][0] = gb;
        gcov2.m[1][1] = gcv;
        // cov2 = X * Tm ; X = Tm^T * Sigma^T
        M3<T> gX = zero3<T>(), gTm = zero3<T>();
        matmul_vjp(st.X, st.Tm, gcov2, gX, gTm);
        M3<T> gTmT = zero3<T>(), gSigmaT = zero3<T>();
        matmul_vjp(transpose(st.Tm), transpose(st.Sigma), gX, gTmT, gSigmaT);
        gTm = [&] {
            M3<T> r = gTm;
            for (int i = 0; i < 3; ++i)
                for (int j = 0; j < 3; ++j) r.m[i][j] += gTmT.m[j][i];
            return r;
        }();
        M3<T> gSigma = transpose(gSigmaT);
        // Tm = W * J
        M3<T> gW = zero3<T>(), gJ = zero3<T>();
        matmul_vjp(st.W, st.J, gTm, gW, gJ);
        // Sigma = M^T * M
        M3<T> gMT = zero3<T>(), gM = zero3<T>();
        matmul_vjp(transpose(st.M), st.M, gSigma, gMT, gM);
        for (int i = 0; i < 3; ++i)
            for (int j = 0; j < 3; ++j) gM.m[i][j] += gMT.m[j][i];
        // M = S * R (S diagonal)
        M3<T> gR;
        for (int i = 0; i < 3; ++i) {
            T acc = T(0);
            for (int j = 0; j < 3; ++j) {
                acc += gM.m[i][j] * st.R.m[i][j];
                gR.m[i][j] = s[i] * gM.m[i][j];
            }
            g.scale[i] = acc;
        }
        // splatting/math.py:13-28 adj_reference_rotation.
        {
            const T r = q[0], x = q[1], y = q[2], z = q[3];
            const auto& G = gR.m;
            g.quat[0] = T(2) * (z * (G[0][1] - G[1][0]) + y * (G[2][0] - G[0][2]) + x * (G[1][2] - G[2][1]));
            g.quat[1] = T(2) * (y * (G[0][1] + G[1][0]) + z * (G[0][2] + G[2][0]) + r * (G[1][2] - G[2][1])) -
                        T(4) * x * (G[1][1] + G[2][2]);
            g.quat[2] = T(2) * (x * (G[0][1] + G[1][0]) + r * (G[2][0] - G[0][2]) + z * (G[1][2] + G[2][1])) -
                        T(4) * y * (G[0][0] + G[2][2]);
            g.quat[3] = T(2) * (r * (G[0][1] - G[1][0]) + x * (G[0][2] + G[2][0]) + y * (G[1][2] + G[2][1])) -
                        T(4) * z * (G[0][0] + G[1][1]);
        }
        // W[i][j] = V[j][i]
        for (int i = 0; i < 3; ++i)
            for (int j = 0; j < 3; ++j) g.view[j][i] += gW.m[i][j];
        // J entries depend on the clamped point t.
        const T* t = st.t;
        T gt[3];
        const T tz2 = t[2] * t[2];
        gt[0] = gJ.m[2][0] * (-fx / tz2);
        gt[1] = gJ.m[2][1] * (-fy / tz2);
        gt[2] = gJ.m[0][0] * (-fx / tz2) + gJ.m[1][1] * (-fy / tz2) +
                gJ.m[2][0] * (T(2) * fx * t[0] / (tz2 * t[2])) +
                gJ.m[2][1] * (T(2) * fy * t[1] / (tz2 * t[2]));
        // splatting/geometry.py:42-51 adj_clamp_point.
        const T xr = pos[0] / pos[2], yr = pos[1] / pos[2];
        T gpos[3];
        gpos[0] = gt[0] * T(xr >= -st.limx && xr <= st.limx ? 1 : 0);
        gpos[1] = gt[1] * T(yr >= -st.limy && yr <= st.limy ? 1 : 0);
        gpos[2] = gt[2];
        // pos = V * [mean, 1] (rows 0..2)
        for (int r = 0; r < 3; ++r) {
            for (int c = 0; c < 3; ++c) {
                g.mean[c] += gpos[r] * V.m[r][c];
                g.view[r][c] += gpos[r] * mean[c];
            }
            g.view[r][3] += gpos[r];
        }
    }
    // Centre path, splatting/geometry.py:106-123.
    {
        T clip[4];
        for (int r = 0; r < 4; ++r) clip[r] = point_row(P, r, mean);
        const T inv_w = T(1) / (clip[3] + T(0.0000001));
        const T gnx = gc[0] * (T(0.5) * T(width));
        const T gny = gc[1] * (T(0.5) * T(height));
        T gclip[4];
        gclip[0] = gnx * inv_w;
        gclip[1] = gny * inv_w;
        gclip[2] = T(0);
        const T ginv = gnx * clip[0] + gny * clip[1];
        gclip[3] = -ginv * inv_w * inv_w;
        for (int r = 0; r < 4; ++r) {
            for (int c = 0; c < 3; ++c) {
                g.mean[c] += gclip[r] * P.m[r][c];
                g.proj[r][c] += gclip[r] * mean[c];
            }
            g.proj[r][3] += gclip[r];
        }
    }
}

// Differentiable scalar projection_loss (gs3d/projection.py:198-210), used
// only by the float64 finite-difference tests.
template <class T>
T projection_loss(const T mean[3], const T q[4], const T s[3], T opacity, const M4<T>& V,
                  const M4<T>& P, int width, int height, T fx, T fy, const T gc[2], const T gk[4]) {
    T pos[3];
    for (int r = 0; r < 3; ++r) pos[r] = point_row(V, r, mean);
    CovState<T> st;
    T cov[3], inv[3];
    screen_covariance<T>(pos, q, s, V, width, height, fx, fy, st, cov);
    invert_covariance<T>(cov, inv);
    T clip[4];
    for (int r = 0; r < 4; ++r) clip[r] = point_row(P, r, mean);
    const T inv_w = T(1) / (clip[3] + T(0.0000001));
    const T cx = ((clip[0] * inv_w + T(1)) * T(width) - T(1)) * T(0.5);
    const T cy = ((clip[1] * inv_w + T(1)) * T(height) - T(1)) * T(0.5);
    return cx * gc[0] + cy * gc[1] + inv[0] * gk[0] + inv[1] * gk[1] + inv[2] * gk[2] + opacity * gk[3];
}

// ---------------------------------------------------------------------------
// Blending helpers shared by forward and backward (gs3d/render.py:85-108,
// :276-290).  The reference leaves contraction to the CUDA compiler; the
// fixed choice here is
//   power = fma(-0.5, fma(c0*dx, dx, (c2*dy)*dy), -((c1*dx)*dy))
//   colour = fma(f, alpha*T, colour)
// ---------------------------------------------------------------------------
inline float blend_power(const float conic[4], float dx, float dy) {
    const float q = fmaf(conic[0] * dx, dx, (conic[2] * dy) * dy);
    return fmaf(-0.5f, q, -((conic[1] * dx) * dy));
}

int g_threads = 1;

// Accumulation shared between threads (render backward, camera gradients).
inline void acc(float* p, float v) {
#pragma omp atomic
    *p += v;
}

}  // namespace

extern "C" {

int oracle_abi_version(void) { return 1; }

// Threads used by the per-Gaussian and per-pixel loops.  With 1 thread every
// accumulation happens in a fixed order (deterministic results).
int oracle_set_threads(int n) {
    g_threads = n < 1 ? 1 : n;
    return g_threads;
}

// ---------------------------------------------------------------------------
// splatting/camera_kernels.py:11-66 prepare_kernel (no contraction).
// ---------------------------------------------------------------------------
int oracle_camera_prepare(const float* views, const float* Ks, int32_t count, int32_t width,
                          int32_t height, int32_t with_centers, float* full, float* inverse,
                          float* centers, int32_t* errors) {
    for (int i = 0; i < count; ++i) {
        const float* K = Ks + 9 * i;
        const float* V = views + 16 * i;
        bool finite = true;
        for (int e = 0; e < 9; ++e) finite = finite && std::isfinite(K[e]);
        int error = 0;
        if (!finite || K[0] <= 0.0f || K[4] <= 0.0f)
            error = 2;
        else if (K[1] != 0.0f || K[3] != 0.0f || K[6] != 0.0f || K[7] != 0.0f || K[8] != 1.0f)
            error = 1;
        errors[i] = error;
        if (error) continue;
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
            // wp.determinant / wp.inverse: cofactor expansion (adjugate / det).
            const float* m = V;
            float inv[16];
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
            const float det = m[0] * inv[0] + m[1] * inv[4] + m[2] * inv[8] + m[3] * inv[12];
            if (det == 0.0f) {
                errors[i] = 3;
                continue;
            }
            const float rdet = 1.0f / det;
            for (int e = 0; e < 16; ++e) inverse[16 * i + e] = inv[e] * rdet;
            for (int r = 0; r < 3; ++r) centers[3 * i + r] = inverse[16 * i + 4 * r + 3];
        }
    }
    return 0;
}

// splatting/camera_kernels.py:69-106 backward_kernel.
int oracle_camera_backward(const float* Ks, const float* grad_full, int32_t width, int32_t height,
                           const float* inverse, const float* grad_centers, int32_t count,
                           float* grad_views) {
    for (int i = 0; i < count; ++i) {
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
    return 0;
}

// gs3d/projection.py:89-164 (+ primitives/sh.py:44-79, splatting/metadata.py:12-31).
int oracle_project_fwd(const gs3d_project_args* a) {
    const int64_t n = a->n;
    for (int v = 0; v < a->views; ++v) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
        for (int64_t i = 0; i < n; ++i) {
            const int64_t row = v * n + i;
            ProjOut o;
            float qn[4];
            const float* q = a->quats + 4 * i;
            if (a->normalize_quats) {
                normalize_quat(q, qn);
                q = qn;
            }
            const bool vis = project_one(a->means + 3 * i, q, a->scales + 3 * i, a->opacities[i],
                                         a->view + 16 * v, a->projection + 16 * v, a->intrinsics + 9 * v, a->width,
                                         a->height, a->near_plane, a->far_plane, a->radius_clip, o, a->tile_mode);
            a->centers[2 * row] = o.center[0];
            a->centers[2 * row + 1] = o.center[1];
            for (int k = 0; k < 4; ++k) a->conics[4 * row + k] = o.conic[k];
            a->radii[row] = o.radius;
            a->tiles[row] = o.tiles;
            a->depths[row] = o.depth;
            if (a->sh) {
                const float* coef = a->sh + v * a->sh_view_stride + (int64_t)3 * a->sh_rows * i;
                float dir[3] = {0.0f, 0.0f, 0.0f};
                if (a->sh_degree > 0)
                    for (int k = 0; k < 3; ++k) dir[k] = a->means[3 * i + k] - a->camera_centers[3 * v + k];
                float color[3], raw[3];
                sh_eval(coef, dir, a->sh_degree, vis, color, raw);
                for (int k = 0; k < 3; ++k) a->colors[3 * row + k] = color[k];
            }
            if (a->means2d) {
                a->means2d[2 * row] = vis ? o.center[0] : 0.0f;
                a->means2d[2 * row + 1] = vis ? o.center[1] : 0.0f;
                a->meta_opacities[row] = vis ? o.conic[3] : 0.0f;
                for (int k = 0; k < 3; ++k) a->meta_conics[3 * row + k] = vis ? o.conic[k] : 0.0f;
            }
        }
    }
    return 0;
}

// primitives/sh.py:44-79 standalone.
int oracle_sh_fwd(const float* coefficients, int32_t rows, const float* directions, const int32_t* radii,
                  int32_t n, int32_t degree, float* colors, uint8_t* active) {
    for (int64_t i = 0; i < n; ++i) {
        const bool vis = radii ? radii[i] > 0 : true;
        float color[3], raw[3];
        sh_eval(coefficients + (int64_t)3 * rows * i, directions + 3 * i, degree, vis, color, raw);
        for (int k = 0; k < 3; ++k) {
            colors[3 * i + k] = color[k];
            if (active) active[3 * i + k] = (vis && raw[k] >= 0.0f) ? 1 : 0;
        }
    }
    return 0;
}

// primitives/sh.py:82-138 standalone.
int oracle_sh_bwd(const float* coefficients, int32_t rows, const float* directions, const int32_t* radii,
                  const uint8_t* active, const float* upstream, int32_t n, int32_t degree,
                  float* grad_coefficients, float* grad_directions) {
    for (int64_t i = 0; i < n; ++i) {
        const bool vis = radii ? radii[i] > 0 : true;
        const bool act[3] = {active[3 * i] != 0, active[3 * i + 1] != 0, active[3 * i + 2] != 0};
        float gd[3];
        sh_backward_row(coefficients + (int64_t)3 * rows * i, directions + 3 * i, degree, vis, act, upstream + 3 * i,
                        grad_coefficients ? grad_coefficients + (int64_t)3 * rows * i : nullptr, rows, gd);
        if (grad_directions)
            for (int k = 0; k < 3; ++k) grad_directions[3 * i + k] = gd[k];
    }
    return 0;
}

// Running error analysis of oracle_sh_bwd (exact upstream gradients):
// [p, r] per entry of the (N,rows,3) coefficient and (N,3) direction
// gradients.
int oracle_sh_bwd_bound(const float* coefficients, int32_t rows, const float* directions, const int32_t* radii,
                        const uint8_t* active, const float* upstream, int32_t n, int32_t degree, double* b_coefficients,
                        double* b_directions) {
    std::vector<Err> gco(3 * rows);
    for (int64_t i = 0; i < n; ++i) {
        const bool vis = radii ? radii[i] > 0 : true;
        const bool act[3] = {active[3 * i] != 0, active[3 * i + 1] != 0, active[3 * i + 2] != 0};
        const Err up[3] = {Err(upstream[3 * i]), Err(upstream[3 * i + 1]), Err(upstream[3 * i + 2])};
        Err gd[3];
        sh_backward_row(coefficients + (int64_t)3 * rows * i, directions + 3 * i, degree, vis, act, up, gco.data(),
                        rows, gd);
        for (int e = 0; b_coefficients && e < 3 * rows; ++e) {
            b_coefficients[2 * ((int64_t)3 * rows * i + e)] = gco[e].p;
            b_coefficients[2 * ((int64_t)3 * rows * i + e) + 1] = gco[e].r;
        }
        for (int k = 0; b_directions && k < 3; ++k) {
            b_directions[2 * (3 * i + k)] = gd[k].p;
            b_directions[2 * (3 * i + k) + 1] = gd[k].r;
        }
    }
    return 0;
}

// gs3d/projection.py:213-285 (+ primitives/sh.py:82-138 and the
// means - centre VJP of gs3d/api.py:160-164).  Sequential accumulation.
int oracle_project_bwd(const gs3d_project_bwd_args* a) {
    const int64_t n = a->n;
    const int K = a->sh_rows;
    if (a->grad_sh) {
        const int64_t per = a->sh_view_stride ? a->sh_view_stride * a->views : (int64_t)3 * K * n;
        std::fill(a->grad_sh, a->grad_sh + per, 0.0f);
    }
    // Camera gradients sum one term per visible Gaussian; the sums are
    // carried in double and rounded once (see RenderGradSink).
    std::vector<double> sum_view(a->grad_view ? 16 * a->views : 0), sum_proj(a->grad_projection ? 16 * a->views : 0);
    std::vector<double> sum_cc(a->grad_camera_centers ? 3 * a->views : 0);
    auto dacc = [](double* p, double v) {
#pragma omp atomic
        *p += v;
    };
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int64_t i = 0; i < n; ++i) {
        float gco[3 * 64];
        double gm[3] = {0, 0, 0}, gq[4] = {0, 0, 0, 0}, gs[3] = {0, 0, 0}, go = 0;
        float qn[4], qnorm = 1.0f;
        const float* quat = a->quats + 4 * i;
        if (a->normalize_quats) {
            qnorm = normalize_quat(quat, qn);
            quat = qn;
        }
        for (int v = 0; v < a->views; ++v) {
            const int64_t row = v * n + i;
            if (a->radii[row] > 0) {
                const M4<float> V = load44<float>(a->view + 16 * v);
                const M4<float> P = load44<float>(a->projection + 16 * v);
                const float* gcp = a->grad_centers + row * a->grad_centers_stride;
                const float* gkp = a->grad_conics + row * a->grad_conics_stride;
                const float gc[2] = {gcp[0], gcp[1]};
                const float gk[4] = {gkp[0], gkp[1], gkp[2], gkp[3]};
                ProjGrad<float> g;
                projection_vjp<float>(a->means + 3 * i, quat, a->scales + 3 * i, a->opacities[i], V, P,
                                      a->width, a->height, a->intrinsics[9 * v], a->intrinsics[9 * v + 4], gc, gk, g);
                for (int k = 0; k < 3; ++k) gm[k] += g.mean[k];
                for (int k = 0; k < 4; ++k) gq[k] += g.quat[k];
                for (int k = 0; k < 3; ++k) gs[k] += g.scale[k];
                go += g.opacity;
                if (a->grad_view)
                    for (int r = 0; r < 4; ++r)
                        for (int c = 0; c < 4; ++c) dacc(&sum_view[16 * v + 4 * r + c], g.view[r][c]);
                if (a->grad_projection)
                    for (int r = 0; r < 4; ++r)
                        for (int c = 0; c < 4; ++c) dacc(&sum_proj[16 * v + 4 * r + c], g.proj[r][c]);
            }
            if (a->sh) {
                const float* coef = a->sh + v * a->sh_view_stride + (int64_t)3 * K * i;
                const bool vis = a->radii[row] > 0;
                float dir[3] = {0.0f, 0.0f, 0.0f};
                if (a->sh_degree > 0)
                    for (int k = 0; k < 3; ++k) dir[k] = a->means[3 * i + k] - a->camera_centers[3 * v + k];
                float color[3], raw[3];
                sh_eval(coef, dir, a->sh_degree, vis, color, raw);
                const bool act[3] = {vis && raw[0] >= 0.0f, vis && raw[1] >= 0.0f, vis && raw[2] >= 0.0f};
                const float* gcol = a->grad_colors + row * a->grad_colors_stride;
                const float up[3] = {gcol[0], gcol[1], gcol[2]};
                float gd[3];
                sh_backward_row(coef, dir, a->sh_degree, vis, act, up, gco, K, gd);
                if (a->grad_sh) {
                    float* dst = a->grad_sh + v * a->sh_view_stride + (int64_t)3 * K * i;
                    for (int e = 0; e < 3 * K; ++e) dst[e] += gco[e];
                }
                if (a->sh_degree > 0) {
                    for (int k = 0; k < 3; ++k) gm[k] += gd[k];
                    if (a->grad_camera_centers)
                        for (int k = 0; k < 3; ++k) dacc(&sum_cc[3 * v + k], -gd[k]);
                }
            }
        }
        if (a->grad_means)
            for (int k = 0; k < 3; ++k) a->grad_means[3 * i + k] = (float)gm[k];
        if (a->grad_quats) {
            float g4[4] = {(float)gq[0], (float)gq[1], (float)gq[2], (float)gq[3]};
            if (a->normalize_quats) normalize_quat_vjp(quat, qnorm, g4);
            for (int k = 0; k < 4; ++k) a->grad_quats[4 * i + k] = g4[k];
        }
        if (a->grad_scales)
            for (int k = 0; k < 3; ++k) a->grad_scales[3 * i + k] = (float)gs[k];
        if (a->grad_opacities) a->grad_opacities[i] = (float)go;
    }
    for (size_t k = 0; k < sum_view.size(); ++k) a->grad_view[k] += (float)sum_view[k];
    for (size_t k = 0; k < sum_proj.size(); ++k) a->grad_projection[k] += (float)sum_proj[k];
    for (size_t k = 0; k < sum_cc.size(); ++k) a->grad_camera_centers[k] += (float)sum_cc[k];
    return 0;
}

// Running error analysis of oracle_project_bwd (see Err).  Inputs: the
// forward data of `a` (exact) and the upstream gradients' values in `a`
// with error bounds e_centers (views,N,2), e_conics (views,N,4) and, with
// SH, e_colors (views,N,3) (bounds on their difference between two
// evaluations; NULL = exact).  Outputs (any may be NULL): per-Gaussian
// [p, r] pairs for means (N,3), quats (N,4), scales (N,3), opacities (N)
// and SH coefficients (grad_sh layout); for the camera sums over Gaussians
// [sum |t|, sum p, sum r, count] per entry of grad_view (views,16),
// grad_projection (views,16) and grad_camera_centers (views,3).
int oracle_project_bwd_bound(const gs3d_project_bwd_args* a, const double* e_centers, const double* e_conics,
                             const double* e_colors, double* b_means, double* b_quats, double* b_scales,
                             double* b_opacities, double* b_sh, double* s_view, double* s_proj, double* s_cc) {
    const int64_t n = a->n;
    const int K = a->sh_rows;
    auto put2 = [](double* dst, const Err& t) {
        dst[0] = t.p;
        dst[1] = t.r;
    };
    auto sum4 = [](double* dst, const Err& t) {
#pragma omp atomic
        dst[0] += ad(t.v);
#pragma omp atomic
        dst[1] += t.p;
#pragma omp atomic
        dst[2] += t.r;
#pragma omp atomic
        dst[3] += 1.0;
    };
    if (b_sh) {
        const int64_t per = a->sh_view_stride ? a->sh_view_stride * a->views : (int64_t)3 * K * n;
        std::fill(b_sh, b_sh + 2 * per, 0.0);
    }
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int64_t i = 0; i < n; ++i) {
        std::vector<Err> gco(3 * K), shsum(a->sh && a->sh_view_stride == 0 ? 3 * K : 0, Err(0.0f));
        Err gm[3] = {Err(0.0f), Err(0.0f), Err(0.0f)}, gq[4] = {Err(0.0f), Err(0.0f), Err(0.0f), Err(0.0f)};
        Err gs[3] = {Err(0.0f), Err(0.0f), Err(0.0f)}, go = Err(0.0f);
        float qn[4], qnorm = 1.0f;
        const float* quat = a->quats + 4 * i;
        if (a->normalize_quats) {
            qnorm = normalize_quat(quat, qn);
            quat = qn;
        }
        Err mean[3], q[4], sc[3];
        for (int k = 0; k < 3; ++k) mean[k] = Err(a->means[3 * i + k]);
        for (int k = 0; k < 4; ++k) q[k] = Err(quat[k]);
        for (int k = 0; k < 3; ++k) sc[k] = Err(a->scales[3 * i + k]);
        for (int v = 0; v < a->views; ++v) {
            const int64_t row = v * n + i;
            if (a->radii[row] > 0) {
                const M4<Err> V = load44<Err>(a->view + 16 * v);
                const M4<Err> P = load44<Err>(a->projection + 16 * v);
                const float* gcp = a->grad_centers + row * a->grad_centers_stride;
                const float* gkp = a->grad_conics + row * a->grad_conics_stride;
                Err gc[2], gk[4];
                for (int k = 0; k < 2; ++k) gc[k] = Err(gcp[k], e_centers ? e_centers[2 * row + k] : 0.0, 0.0);
                for (int k = 0; k < 4; ++k) gk[k] = Err(gkp[k], e_conics ? e_conics[4 * row + k] : 0.0, 0.0);
                ProjGrad<Err> g;
                projection_vjp<Err>(mean, q, sc, Err(a->opacities[i]), V, P, a->width, a->height,
                                    Err(a->intrinsics[9 * v]), Err(a->intrinsics[9 * v + 4]), gc, gk, g);
                for (int k = 0; k < 3; ++k) gm[k] += g.mean[k];
                for (int k = 0; k < 4; ++k) gq[k] += g.quat[k];
                for (int k = 0; k < 3; ++k) gs[k] += g.scale[k];
                go += g.opacity;
                for (int r = 0; r < 4; ++r)
                    for (int c = 0; c < 4; ++c) {
                        if (s_view) sum4(s_view + 4 * (16 * v + 4 * r + c), g.view[r][c]);
                        if (s_proj) sum4(s_proj + 4 * (16 * v + 4 * r + c), g.proj[r][c]);
                    }
            }
            if (a->sh) {
                const float* coef = a->sh + v * a->sh_view_stride + (int64_t)3 * K * i;
                const bool vis = a->radii[row] > 0;
                float dir[3] = {0.0f, 0.0f, 0.0f};
                if (a->sh_degree > 0)
                    for (int k = 0; k < 3; ++k) dir[k] = a->means[3 * i + k] - a->camera_centers[3 * v + k];
                float color[3], raw[3];
                sh_eval(coef, dir, a->sh_degree, vis, color, raw);
                const bool act[3] = {vis && raw[0] >= 0.0f, vis && raw[1] >= 0.0f, vis && raw[2] >= 0.0f};
                const float* gcol = a->grad_colors + row * a->grad_colors_stride;
                Err up[3];
                for (int k = 0; k < 3; ++k) up[k] = Err(gcol[k], e_colors ? e_colors[3 * row + k] : 0.0, 0.0);
                Err gd[3];
                sh_backward_row(coef, dir, a->sh_degree, vis, act, up, gco.data(), K, gd);
                if (b_sh) {
                    if (a->sh_view_stride == 0) {
                        for (int e = 0; e < 3 * K; ++e) shsum[e] += gco[e];
                    } else {
                        double* dst = b_sh + 2 * (v * a->sh_view_stride + (int64_t)3 * K * i);
                        for (int e = 0; e < 3 * K; ++e) put2(dst + 2 * e, gco[e]);
                    }
                }
                if (a->sh_degree > 0) {
                    for (int k = 0; k < 3; ++k) gm[k] += gd[k];
                    if (s_cc)
                        for (int k = 0; k < 3; ++k) sum4(s_cc + 4 * (3 * v + k), -gd[k]);
                }
            }
        }
        if (b_sh && a->sh_view_stride == 0)
            for (int e = 0; e < 3 * K; ++e) put2(b_sh + 2 * ((int64_t)3 * K * i + e), shsum[e]);
        if (b_means)
            for (int k = 0; k < 3; ++k) put2(b_means + 2 * (3 * i + k), gm[k]);
        if (b_quats) {
            if (a->normalize_quats) normalize_quat_vjp(quat, qnorm, gq);
            for (int k = 0; k < 4; ++k) put2(b_quats + 2 * (4 * i + k), gq[k]);
        }
        if (b_scales)
            for (int k = 0; k < 3; ++k) put2(b_scales + 2 * (3 * i + k), gs[k]);
        if (b_opacities) put2(b_opacities + 2 * i, go);
    }
    return 0;
}

// Running error analysis of oracle_camera_backward: grad_full and
// grad_centers with error bounds e_full (count,16) and e_centers (count,3)
// (NULL = exact); writes [p, r] per entry of the (count,4,4) result.
int oracle_camera_backward_bound(const float* Ks, const float* grad_full, const double* e_full, int32_t width,
                                 int32_t height, const float* inverse, const float* grad_centers,
                                 const double* e_centers, int32_t count, double* out) {
    for (int i = 0; i < count; ++i) {
        const float* K = Ks + 9 * i;
        const Err px = Err(2.0f * K[0] / (float)width), py = Err(2.0f * K[4] / (float)height);
        const Err cx = Err(2.0f * K[2] / (float)width - 1.0f), cy = Err(2.0f * K[5] / (float)height - 1.0f);
        Err G[16], gcen[3];
        for (int k = 0; k < 16; ++k)
            G[k] = grad_full ? Err(grad_full[16 * i + k], e_full ? e_full[16 * i + k] : 0.0, 0.0) : Err(0.0f);
        for (int k = 0; k < 3; ++k)
            gcen[k] = grad_centers ? Err(grad_centers[3 * i + k], e_centers ? e_centers[3 * i + k] : 0.0, 0.0)
                                   : Err(0.0f);
        for (int row = 0; row < 4; ++row)
            for (int col = 0; col < 4; ++col) {
                Err value = Err(0.0f);
                if (grad_full) {
                    if (row == 0)
                        value = px * G[col];
                    else if (row == 1)
                        value = py * G[4 + col];
                    else if (row == 2)
                        value = (cx * G[col] + cy * G[4 + col]) + G[8 + col] + G[12 + col];
                }
                if (grad_centers) {
                    const float* inv = inverse + 16 * i;
                    Err vjp = Err(0.0f);
                    for (int k = 0; k < 3; ++k) vjp += Err(inv[4 * k + row]) * gcen[k];
                    value -= vjp * Err(inv[4 * col + 3]);
                }
                out[2 * (16 * i + 4 * row + col)] = value.p;
                out[2 * (16 * i + 4 * row + col) + 1] = value.r;
            }
    }
    return 0;
}

// float64 instantiations for finite-difference tests of the VJP.
double oracle_projection_loss_f64(const double* mean, const double* quat, const double* scale, double opacity,
                                  const double* view, const double* proj, int32_t width, int32_t height, double fx,
                                  double fy, const double* gc, const double* gk) {
    M4<double> V, P;
    for (int i = 0; i < 16; ++i) {
        V.m[i / 4][i % 4] = view[i];
        P.m[i / 4][i % 4] = proj[i];
    }
    return projection_loss<double>(mean, quat, scale, opacity, V, P, width, height, fx, fy, gc, gk);
}

int oracle_projection_vjp_f64(const double* mean, const double* quat, const double* scale, double opacity,
                              const double* view, const double* proj, int32_t width, int32_t height, double fx,
                              double fy, const double* gc, const double* gk, double* out /* 3+4+3+1+16+16 */) {
    M4<double> V, P;
    for (int i = 0; i < 16; ++i) {
        V.m[i / 4][i % 4] = view[i];
        P.m[i / 4][i % 4] = proj[i];
    }
    ProjGrad<double> g;
    projection_vjp<double>(mean, quat, scale, opacity, V, P, width, height, fx, fy, gc, gk, g);
    int o = 0;
    for (int k = 0; k < 3; ++k) out[o++] = g.mean[k];
    for (int k = 0; k < 4; ++k) out[o++] = g.quat[k];
    for (int k = 0; k < 3; ++k) out[o++] = g.scale[k];
    out[o++] = g.opacity;
    for (int r = 0; r < 4; ++r)
        for (int c = 0; c < 4; ++c) out[o++] = g.view[r][c];
    for (int r = 0; r < 4; ++r)
        for (int c = 0; c < 4; ++c) out[o++] = g.proj[r][c];
    return 0;
}

// Forward intermediates for the custom-adjoint known-answer tests.
float oracle_expf(float x) { return gs_expf(x); }

float oracle_logf(float x) { return gs_logf(x); }

// Normalised quaternions u and gradients through the normalisation of count
// raw quaternions q with upstream gradients g (g and grad may be NULL).
int oracle_normalize_quats(const float* q, int64_t count, float* u, const float* g, float* grad) {
    for (int64_t i = 0; i < count; ++i) {
        const float norm = normalize_quat(q + 4 * i, u + 4 * i);
        if (g && grad) {
            float gi[4] = {g[4 * i], g[4 * i + 1], g[4 * i + 2], g[4 * i + 3]};
            normalize_quat_vjp(u + 4 * i, norm, gi);
            for (int k = 0; k < 4; ++k) grad[4 * i + k] = gi[k];
        }
    }
    return 0;
}

int oracle_tile_footprint(int32_t mode, const float* center, const float* conic, int32_t radius, int32_t gx,
                          int32_t gy, int64_t* tiles, int32_t* bounds) {
    Ellipse e;
    tile_bounds(center, radius, gx, gy, e.bounds);
    if (mode != GS3D_TILE_RADIUS) e = footprint(center, conic, radius, gx, gy);
    if (bounds)
        for (int k = 0; k < 4; ++k) bounds[k] = e.bounds[k];
    return visit_tiles(mode, center, conic, radius, gx, gy, tiles);
}

int oracle_glm_rotation(const float* q, float* out) {
    M3<float> R = glm_rotation<float>(q);
    for (int i = 0; i < 9; ++i) out[i] = R.m[i / 3][i % 3];
    return 0;
}

// SH basis / gradient access for tests.
float oracle_sh_basis(const float* u, int32_t k) { return sh_basis(u, k); }
int oracle_sh_basis_grad(const float* u, int32_t k, float* g) {
    sh_basis_grad(u, k, g);
    return 0;
}

// primitives/tiling.py:57-64 scan_counts (inclusive), 64-bit total.
int oracle_scan_i32(const int32_t* counts, int64_t n, int32_t* offsets, int64_t* total) {
    int64_t s = 0;
    for (int64_t i = 0; i < n; ++i) {
        s += counts[i];
        offsets[i] = (int32_t)s;
    }
    if (total) *total = s;
    return 0;
}

// splatting/binning.py:16-37 duplicate (:40-68 duplicate_precise for the
// SnugBox/AccuTile modes) + primitives/tiling.py:32-36 sort_key.
int oracle_emit_keys(const gs3d_emit_args* a) {
    const int gx = (a->width + 15) / 16, gy = (a->height + 15) / 16;
    const int64_t tiles_per_view = (int64_t)gx * gy;
    const int64_t rows = (int64_t)a->n * a->views;
    std::vector<int64_t> tiles;
    for (int64_t r = 0; r < rows; ++r) {
        if (a->radii[r] <= 0) continue;
        const int64_t v = r / a->n;
        if (a->tile_mode != GS3D_TILE_RADIUS) {
            tiles.resize((size_t)gx * gy);
            const int count = visit_tiles(a->tile_mode, a->centers + 2 * r, a->conics + 4 * r, a->radii[r], gx, gy,
                                          tiles.data());
            const int64_t off = r > 0 ? a->offsets[r - 1] : 0;
            uint32_t bits;
            std::memcpy(&bits, a->depths + r, 4);
            for (int k = 0; k < count; ++k) {
                const uint64_t tile = (uint64_t)(uint32_t)(v * tiles_per_view + tiles[k]);
                a->keys[off + k] = (tile << 32) | (uint64_t)bits;
                a->values[off + k] = (int32_t)(r % a->n);
            }
            continue;
        }
        int b[4];
        tile_bounds(a->centers + 2 * r, a->radii[r], gx, gy, b);
        int64_t off = r > 0 ? a->offsets[r - 1] : 0;
        uint32_t bits;
        std::memcpy(&bits, a->depths + r, 4);
        for (int y = b[1]; y < b[3]; ++y)
            for (int x = b[0]; x < b[2]; ++x) {
                const uint64_t tile = (uint64_t)(uint32_t)(v * tiles_per_view + y * gx + x);
                a->keys[off] = (tile << 32) | (uint64_t)bits;
                a->values[off] = (int32_t)(r % a->n);
                ++off;
            }
    }
    return 0;
}

// primitives/tiling.py:67-86: stable sort on key bits [0, end_bit).  Sorting
// (masked key, input position) pairs, which are all distinct, gives exactly
// the stable order; the parallel sort then needs no stability of its own.
int oracle_sort_pairs_u64(uint64_t* keys, int32_t* values, int64_t count, int32_t end_bit) {
    const uint64_t mask = end_bit >= 64 ? ~0ull : ((1ull << end_bit) - 1ull);
    struct Item {
        uint64_t key;
        int64_t pos;
        bool operator<(const Item& o) const { return key < o.key || (key == o.key && pos < o.pos); }
    };
    std::vector<Item> items(count);
    for (int64_t i = 0; i < count; ++i) items[i] = Item{keys[i] & mask, i};
    if (g_threads > 1) {
        omp_set_num_threads(g_threads);
        __gnu_parallel::sort(items.begin(), items.end());
    } else {
        std::sort(items.begin(), items.end());
    }
    std::vector<uint64_t> k2(count);
    std::vector<int32_t> v2(count);
    for (int64_t i = 0; i < count; ++i) {
        k2[i] = keys[items[i].pos];
        v2[i] = values[items[i].pos];
    }
    std::copy(k2.begin(), k2.end(), keys);
    std::copy(v2.begin(), v2.end(), values);
    return 0;
}

// primitives/tiling.py:39-54 identify_ranges.
int oracle_tile_ranges(const uint64_t* keys, int64_t count, int32_t* ranges, int64_t tile_count) {
    (void)tile_count;
    for (int64_t i = 0; i < count; ++i) {
        const uint32_t cur = (uint32_t)(keys[i] >> 32);
        if (i == 0) {
            if (cur != 0xFFFFFFFFu) ranges[2 * (int64_t)cur] = 0;
        } else {
            const uint32_t prev = (uint32_t)(keys[i - 1] >> 32);
            if (cur != prev) {
                if (prev != 0xFFFFFFFFu) ranges[2 * (int64_t)prev + 1] = (int32_t)i;
                if (cur != 0xFFFFFFFFu) ranges[2 * (int64_t)cur] = (int32_t)i;
            }
        }
        if (i == count - 1 && cur != 0xFFFFFFFFu) ranges[2 * (int64_t)cur + 1] = (int32_t)count;
    }
    return 0;
}

// Assemble the blended vector of one Gaussian (gs3d/autograd.py:41-46).
static inline void gather_features(const gs3d_render_args* a, int v, int64_t g, float* out) {
    int c = 0;
    const float* f = a->features + v * a->feat_view_stride + g * a->feat_stride;
    for (int k = 0; k < a->feat_channels; ++k) out[c++] = f[k];
    if (a->extra_channels) {
        const float* e = a->extra + v * a->extra_view_stride + g * a->extra_stride;
        for (int k = 0; k < a->extra_channels; ++k) out[c++] = e[k];
    }
    if (a->one_tail) out[c++] = 1.0f;
}

static inline int total_channels(const gs3d_render_args* a) {
    return a->feat_channels + a->extra_channels + (a->one_tail ? 1 : 0);
}

// statistics.py:46-70 (make_observer), called per accepted blend at
// gs3d/render.py:109-115: request r reads its pixel value; a nonzero value
// adds 1 to the Gaussian's count row, or value * weight to its sum row.  Rows
// number the requests of one kind in request order.
static void observe(const gs3d_render_stats_args* st, int v, int n, int64_t g, int64_t pixel, int64_t plane,
                    float weight) {
    int count_row = 0, sum_row = 0;
    for (int r = 0; r < st->requests; ++r) {
        const float value = st->pixel_values[v * st->pixel_view_stride + r * plane + pixel];
        if ((st->sum_mask >> r) & 1u) {
            if (value != 0.0f) st->sums[v * st->sums_view_stride + (int64_t)sum_row * n + g] += value * weight;
            ++sum_row;
        } else {
            if (value != 0.0f) st->counts[v * st->counts_view_stride + (int64_t)count_row * n + g] += 1;
            ++count_row;
        }
    }
}

// gs3d/render.py:36-126 forward, one pixel at a time.  With statistics the
// pixels run in order on one thread (the observer accumulates).
static int render_fwd(const gs3d_render_args* a, const gs3d_render_stats_args* st, int64_t* pair_counts = nullptr) {
    const int W = a->width, H = a->height;
    const int gx = (W + 15) / 16, gy = (H + 15) / 16;
    const int D = total_channels(a);
    std::vector<float> bg(D);
    const int threads = st ? 1 : g_threads;
    int64_t visited_all = 0, accepted_all = 0;
    for (int v = 0; v < a->views; ++v) {
        for (int k = 0; k < D; ++k)
            bg[k] = (a->background && k < a->feat_channels) ? a->background[v * a->background_view_stride + k] : 0.0f;
#pragma omp parallel for schedule(dynamic, 4) num_threads(threads) reduction(+ : visited_all, accepted_all)
        for (int y = 0; y < H; ++y) {
            std::vector<float> color(D), f(D);
            for (int x = 0; x < W; ++x) {
                const int64_t tile = (int64_t)v * gx * gy + (y / 16) * gx + (x / 16);
                const int first = a->ranges[2 * tile], last = a->ranges[2 * tile + 1];
                float T = 1.0f;
                std::fill(color.begin(), color.end(), 0.0f);
                int contributor = 0, last_contributor = 0;
                for (int idx = first; idx < last; ++idx) {
                    contributor += 1;
                    const int64_t g = a->ids[idx];
                    const int64_t row = (int64_t)v * a->n + g;
                    const float dx = a->centers[2 * row] - (float)x;
                    const float dy = a->centers[2 * row + 1] - (float)y;
                    const float* conic = a->conics + 4 * row;
                    const float power = blend_power(conic, dx, dy);
                    if (!(power <= 0.0f)) continue;
                    const float alpha = std::min(0.99f, conic[3] * gs_expf(power));
                    if (!(alpha >= 1.0f / 255.0f)) continue;
                    const float next_t = T * (1.0f - alpha);
                    if (next_t < 0.0001f) break;
                    gather_features(a, v, g, f.data());
                    // gs3d/render.py:106-108 adds value * alpha * transmittance,
                    // i.e. (v * alpha) * T; the kernels and this restatement
                    // reassociate it as v * (alpha * T), one weight per pixel
                    // shared by every channel (at most one rounding of the
                    // product apart per term).
                    const float w = alpha * T;
                    for (int k = 0; k < D; ++k) color[k] = fmaf(f[k], w, color[k]);
                    if (st) observe(st, v, a->n, g, (int64_t)y * W + x, (int64_t)W * H, w);
                    T = next_t;
                    last_contributor = contributor;
                    accepted_all += 1;
                }
                visited_all += contributor;  // entries the loop visited, the terminating one included
                const int64_t pix = ((int64_t)v * H + y) * W + x;
                for (int k = 0; k < D; ++k) a->image[pix * D + k] = fmaf(T, bg[k], color[k]);
                a->final_t[pix] = T;
                a->contributors[pix] = last_contributor;
            }
        }
    }
    if (pair_counts) {
        pair_counts[0] = visited_all;
        pair_counts[1] = accepted_all;
    }
    return 0;
}

int oracle_render_fwd(const gs3d_render_args* a) { return render_fwd(a, nullptr); }

// render_fwd and the (pixel, Gaussian) pairs its loop visits and accepts
// (counts[0], counts[1]).
int oracle_render_pair_counts(const gs3d_render_args* a, int64_t* counts) { return render_fwd(a, nullptr, counts); }

int oracle_render_fwd_stats(const gs3d_render_args* a, const gs3d_render_stats_args* st) { return render_fwd(a, st); }

}  // extern "C"

// gs3d/render.py:211-356 backward, sequential accumulation per pixel in
// tile-then-row-major order (the GPU sums the same terms in another order).
// T is float (the oracle) or Err (the same arithmetic with its running error
// bound); every term goes to sink.add(kind, index, value) with kind 0
// centres (views,N,2), 1 conics (views,N,4), 2 absolute centres (views,N,2),
// 3 features and 4 extra channels (indices in the gradient arrays' layout).
enum { kSinkCenters, kSinkConics, kSinkAbs, kSinkFeatures, kSinkExtra };

template <class T, class Sink>
static void render_bwd_core(const gs3d_render_bwd_args* b, Sink& sink) {
    const gs3d_render_args* a = &b->fwd;
    const int W = a->width, H = a->height;
    const int gx = (W + 15) / 16, gy = (H + 15) / 16;
    const int D = total_channels(a);
    const int Dg = D - (a->one_tail ? 1 : 0);
    std::vector<float> bg(D);
    for (int v = 0; v < a->views; ++v) {
        for (int k = 0; k < D; ++k)
            bg[k] = (a->background && k < a->feat_channels) ? a->background[v * a->background_view_stride + k] : 0.0f;
#pragma omp parallel for schedule(dynamic, 4) num_threads(g_threads)
        for (int y = 0; y < H; ++y) {
            std::vector<T> grad(D), accum(D), last_color(D);
            std::vector<float> f(D);
            for (int x = 0; x < W; ++x) {
                const int64_t tile = (int64_t)v * gx * gy + (y / 16) * gx + (x / 16);
                const int first = a->ranges[2 * tile], last = a->ranges[2 * tile + 1];
                const int64_t pix = ((int64_t)v * H + y) * W + x;
                const float final_T = a->final_t[pix];
                T Tr = T(final_T);
                const int last_contributor = a->contributors[pix];
                T bg_grad = T(0.0f);
                for (int k = 0; k < D; ++k) {
                    grad[k] = T(b->upstream[pix * D + k]);
                    bg_grad += T(bg[k]) * grad[k];
                    accum[k] = T(0.0f);
                    last_color[k] = T(0.0f);
                }
                T last_alpha = T(0.0f);
                int contributor = last - first;
                for (int idx = last - 1; idx >= first; --idx) {
                    contributor -= 1;
                    if (!(contributor < last_contributor)) continue;
                    const int64_t g = a->ids[idx];
                    const int64_t row = (int64_t)v * a->n + g;
                    const float dx = a->centers[2 * row] - (float)x;
                    const float dy = a->centers[2 * row + 1] - (float)y;
                    const float* conic = a->conics + 4 * row;
                    const float power = blend_power(conic, dx, dy);
                    if (!(power <= 0.0f)) continue;
                    const float G = gs_expf(power);
                    const float alpha = std::min(0.99f, conic[3] * G);
                    if (!(alpha >= 1.0f / 255.0f)) continue;
                    Tr = Tr / T(1.0f - alpha);
                    gather_features(a, v, g, f.data());
                    T grad_alpha = T(0.0f);
                    for (int k = 0; k < D; ++k) {
                        accum[k] = last_alpha * last_color[k] + (T(1.0f) - last_alpha) * accum[k];
                        last_color[k] = T(f[k]);
                        grad_alpha += (T(f[k]) - accum[k]) * grad[k];
                        if (k < Dg) {
                            const T gv = T(alpha) * Tr * grad[k];
                            if (k < a->feat_channels)
                                sink.add(kSinkFeatures, v * b->grad_feat_view_stride + g * b->grad_feat_stride + k, gv);
                            else
                                sink.add(kSinkExtra,
                                         v * b->grad_extra_view_stride + g * b->grad_extra_stride + (k - a->feat_channels),
                                         gv);
                        }
                    }
                    grad_alpha = grad_alpha * Tr + T(-final_T / (1.0f - alpha)) * bg_grad;
                    last_alpha = T(alpha);
                    const T gvv = T(conic[3]) * grad_alpha;
                    const float gdx = G * dx, gdy = G * dy;
                    const T dcx = gvv * T(-gdx * conic[0] - gdy * conic[1]);
                    const T dcy = gvv * T(-gdy * conic[2] - gdx * conic[1]);
                    sink.add(kSinkCenters, 2 * row, dcx);
                    sink.add(kSinkCenters, 2 * row + 1, dcy);
                    sink.add(kSinkAbs, 2 * row, dcx);
                    sink.add(kSinkAbs, 2 * row + 1, dcy);
                    sink.add(kSinkConics, 4 * row, T(-0.5f * gdx * dx) * gvv);
                    sink.add(kSinkConics, 4 * row + 1, T(-gdx * dy) * gvv);
                    sink.add(kSinkConics, 4 * row + 2, T(-0.5f * gdy * dy) * gvv);
                    sink.add(kSinkConics, 4 * row + 3, T(G) * grad_alpha);
                }
            }
        }
    }
}

// Sink of the oracle: the reference's atomic adds of the float32 terms into
// the gradient arrays (gs3d/render.py:306-354).  The sums are carried in
// double and rounded once at the end: the reference's atomics add in an
// unspecified order, and one sequential float32 sum of the ~10^6 terms of a
// large Gaussian loses up to 5e-3 of its value (increments below half an ulp
// of the running sum vanish), far more than any order a GPU adds them in.
struct RenderGradSink {
    const gs3d_render_bwd_args* b;
    std::vector<double> sum[5];
    explicit RenderGradSink(const gs3d_render_bwd_args* args) : b(args) {
        const gs3d_render_args& a = b->fwd;
        const int64_t rows = (int64_t)a.views * a.n;
        sum[kSinkCenters].assign(2 * rows, 0.0);
        sum[kSinkConics].assign(4 * rows, 0.0);
        if (b->abs_centers) sum[kSinkAbs].assign(2 * rows, 0.0);
        if (b->grad_features)
            sum[kSinkFeatures].assign(b->grad_feat_view_stride ? a.views * b->grad_feat_view_stride
                                                               : a.n * b->grad_feat_stride, 0.0);
        if (b->grad_extra)
            sum[kSinkExtra].assign(b->grad_extra_view_stride ? a.views * b->grad_extra_view_stride
                                                             : a.n * b->grad_extra_stride, 0.0);
    }
    void add(int kind, int64_t i, float t) {
        if (sum[kind].empty()) return;
        double* d = &sum[kind][i];
        const double v = kind == kSinkAbs ? std::fabs((double)t) : (double)t;
#pragma omp atomic
        *d += v;
    }
    // Adds the rounded sums to the gradient arrays.
    void finish() const {
        for (size_t i = 0; i < sum[kSinkCenters].size(); ++i)
            b->grad_centers[(i / 2) * b->grad_centers_stride + (i % 2)] += (float)sum[kSinkCenters][i];
        for (size_t i = 0; i < sum[kSinkConics].size(); ++i)
            b->grad_conics[(i / 4) * b->grad_conics_stride + (i % 4)] += (float)sum[kSinkConics][i];
        for (size_t i = 0; i < sum[kSinkAbs].size(); ++i)
            b->abs_centers[(i / 2) * b->abs_stride + (i % 2)] += (float)sum[kSinkAbs][i];
        for (size_t i = 0; i < sum[kSinkFeatures].size(); ++i) b->grad_features[i] += (float)sum[kSinkFeatures][i];
        for (size_t i = 0; i < sum[kSinkExtra].size(); ++i) b->grad_extra[i] += (float)sum[kSinkExtra][i];
    }
};

// Sink of the error analysis: per gradient entry, 4 doubles
// [sum |term|, sum p, sum r, number of terms] in dense per-kind arrays
// (centres/abs (views*N*2), conics (views*N*4), features and extra in the
// layout of their gradient arrays).
struct RenderBoundSink {
    double* out[5];
    static void add4(double* q, const Err& t) {
        double* d = q;
#pragma omp atomic
        d[0] += ad(t.v);
#pragma omp atomic
        d[1] += t.p;
#pragma omp atomic
        d[2] += t.r;
#pragma omp atomic
        d[3] += 1.0;
    }
    void add(int kind, int64_t i, const Err& t) const {
        if (out[kind]) add4(out[kind] + 4 * i, kind == kSinkAbs ? Err(std::fabs(t.v), t.p, t.r) : t);
    }
};

// Sink of the float64 evaluation (the same template in double arithmetic,
// the forward decisions still in float32): near-exact gradients against
// which the error bound is checked.
struct RenderF64Sink {
    double* out[5];
    void add(int kind, int64_t i, double t) const {
        if (!out[kind]) return;
        double* d = out[kind] + i;
#pragma omp atomic
        *d += kind == kSinkAbs ? std::fabs(t) : t;
    }
};

extern "C" {

int oracle_render_bwd(const gs3d_render_bwd_args* b) {
    RenderGradSink sink(b);
    render_bwd_core<float>(b, sink);
    sink.finish();
    return 0;
}

// Running error analysis of oracle_render_bwd: for every gradient entry the
// terms' [sum |t|, sum p, sum r, count] (see RenderBoundSink); any of the
// five outputs may be NULL.
int oracle_render_bwd_bound(const gs3d_render_bwd_args* b, double* centers, double* conics, double* abs_centers,
                            double* features, double* extra) {
    RenderBoundSink sink{{centers, conics, abs_centers, features, extra}};
    render_bwd_core<Err>(b, sink);
    return 0;
}

// oracle_render_bwd evaluated in double (dense outputs in the layouts of
// the bound's arrays, one double per entry).
int oracle_render_bwd_f64(const gs3d_render_bwd_args* b, double* centers, double* conics, double* abs_centers,
                          double* features, double* extra) {
    RenderF64Sink sink{{centers, conics, abs_centers, features, extra}};
    render_bwd_core<double>(b, sink);
    return 0;
}


}  // extern "C"
