// SnugBox / AccuTile tile footprints of projected Gaussians
// (splatting/intersections.py:46-218).
//
// footprint(): the opacity-aware ellipse {a dx^2 + 2b dx dy + c dy^2 <= level}
// with level = 2 ln(255 o) plus a float32 rounding allowance, its extents,
// and its tile rectangle clipped to the 3-sigma square (SnugBox).  AccuTile
// walks the rectangle in strips of tiles along its shorter side and keeps,
// per strip, the tiles between the ellipse's extreme points inside the
// strip (strip_span).  Counting and listing use the same strip spans, so
// allocations and the written lists always agree.  Arithmetic follows the
// reference operation by operation in float32 without contraction (the file
// is built with -ffp-contract=off); the natural log is a fixed sequence of
// IEEE double operations, identical on the host and the device.
#pragma once

#include "common.hpp"

namespace gs3d {

// ln(x) rounded to float from IEEE double operations only: x = m 2^e with m
// in [sqrt(1/2), sqrt(2)), ln m = 2 atanh(s), s = (m - 1)/(m + 1)
// (|s| <= 0.1716), atanh by its Taylor series through s^23.
GS3D_DEV float ln_f32(float x) {
    if (!(x >= 0.0f)) return __builtin_nanf("");
    if (x == 0.0f) return -__builtin_inff();
    if (x == __builtin_inff()) return x;
    int e = 0;
    if (x < 1.17549435e-38f) {
        x *= 18446744073709551616.0f;  // 2^64: subnormals into the normal range
        e = -64;
    }
    uint32_t bits = __float_as_uint(x);
    e += (int)(bits >> 23) - 127;
    double m = (double)__uint_as_float((bits & 0x007FFFFFu) | 0x3F800000u);
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

struct Ellipse {
    float cx, cy, a, b, c;
    float level, det, ex, ey;
    int4 bounds;  // x0, y0, x1, y1 (exclusive ends)
    bool precise;
};

GS3D_DEV float floor_clamp(float v, float lo, float hi) { return sel_clamp(__builtin_floorf(v), lo, hi); }

// intersections.py:46-116 footprint.
GS3D_DEV Ellipse footprint(float2 center, float4 conic, int radius, int gx, int gy) {
    Ellipse e;
    e.cx = center.x;
    e.cy = center.y;
    e.a = conic.x;
    e.b = conic.y;
    e.c = conic.z;
    e.level = e.det = e.ex = e.ey = 0.0f;
    e.precise = false;
    e.bounds = tile_rect(center.x, center.y, radius, gx, gy);
    const float a = conic.x, b = conic.y, c = conic.z;
    const float det = (float)((double)a * (double)c - (double)b * (double)b);
    if (conic.w < 1.0f / 255.0f) {
        e.bounds = make_int4(0, 0, 0, 0);
        return e;
    }
    if (!(a > 0.0f && c > 0.0f && det > 0.0f)) return e;
    const float level = 2.0f * ln_f32(conic.w * 255.0f);
    const float reach = (float)radius + 32.0f;
    const float span = ((a + 2.0f * __builtin_fabsf(b)) + c) * reach * reach;
    const float roundoff = 9.5367431640625e-07f * ((span + __builtin_fabsf(level)) + 1.0f);
    e.level = sel_max(0.0f, level) + roundoff;
    e.det = det;
    e.ex = __builtin_sqrtf(e.level * c / det);
    e.ey = __builtin_sqrtf(e.level * a / det);
    if (!(__builtin_isfinite(e.ex) && __builtin_isfinite(e.ey))) return e;
    const int lo_x = (int)floor_clamp((e.cx - e.ex) / 16.0f, 0.0f, (float)gx);
    const int lo_y = (int)floor_clamp((e.cy - e.ey) / 16.0f, 0.0f, (float)gy);
    const int hi_x = (int)sel_clamp(__builtin_floorf((e.cx + e.ex) / 16.0f) + 1.0f, 0.0f, (float)gx);
    const int hi_y = (int)sel_clamp(__builtin_floorf((e.cy + e.ey) / 16.0f) + 1.0f, 0.0f, (float)gy);
    e.bounds = make_int4(max(e.bounds.x, lo_x), max(e.bounds.y, lo_y), min(e.bounds.z, hi_x), min(e.bounds.w, hi_y));
    e.precise = true;
    return e;
}

// intersections.py:119-130: the two crossings of line u = 16 * line (u = y
// for strips of tile rows, x for strips of tile columns).
GS3D_DEV float2 line_intersection(const Ellipse& e, int line, bool is_y) {
    const float u = is_y ? e.cy : e.cx, v = is_y ? e.cx : e.cy;
    const float c = is_y ? e.a : e.c, ext = is_y ? e.ey : e.ex;
    const float h = sel_clamp((float)(line * 16) - u, -ext, ext);
    const float root = __builtin_sqrtf(sel_max(0.0f, e.level * c - e.det * h * h));
    const float bh = -e.b * h;
    return make_float2(v + (bh - root) / c, v + (bh + root) / c);
}

// intersections.py:133-157: [first, end) tiles of strip `row`, given the
// crossings of its two boundary lines.
GS3D_DEV int2 strip_span(const Ellipse& e, int row, bool is_y, float2 low, float2 high) {
    const float u = is_y ? e.cy : e.cx, v = is_y ? e.cx : e.cy;
    const float a = is_y ? e.c : e.a, ext = is_y ? e.ex : e.ey;
    const int lower = is_y ? e.bounds.x : e.bounds.y, upper = is_y ? e.bounds.z : e.bounds.w;
    float lo = sel_min(low.x, high.x), hi = sel_max(low.y, high.y);
    const float arg_min = e.b * ext / a, arg_max = -e.b * ext / a;
    const float h0 = (float)(row * 16) - u, h1 = (float)((row + 1) * 16) - u;
    if (h0 <= arg_min && arg_min <= h1) lo = v - ext;
    if (h0 <= arg_max && arg_max <= h1) hi = v + ext;
    return make_int2((int)floor_clamp(lo / 16.0f, (float)lower, (float)upper),
                     (int)sel_clamp(__builtin_floorf(hi / 16.0f) + 1.0f, (float)lower, (float)upper));
}

// Rectangle of a row in the rectangle modes; for AccuTile, the rectangle its
// strips lie in.
GS3D_DEV int4 mode_rect(float2 center, float4 conic, int radius, int gx, int gy, int mode) {
    if (mode == GS3D_TILE_RADIUS) return tile_rect(center.x, center.y, radius, gx, gy);
    return footprint(center, conic, radius, gx, gy).bounds;
}

// AccuTile traversal (intersections.py:160-218): calls f(strip, first, end)
// for every strip in order; is_y tells whether strips are tile rows (spans
// of x) or tile columns (spans of y).  Returns the number of tiles.
template <class F>
GS3D_DEV int accutile_strips(const Ellipse& e, bool& is_y, F&& f) {
    const int4 b = e.bounds;
    const int nx = max(0, b.z - b.x), ny = max(0, b.w - b.y);
    is_y = ny < nx;
    if (nx == 0 || ny == 0) return 0;
    const int start = is_y ? b.y : b.x, end = is_y ? b.w : b.z;
    const int full0 = is_y ? b.x : b.y, full1 = is_y ? b.z : b.w;
    float2 low = make_float2(0.0f, 0.0f);
    if (e.precise) low = line_intersection(e, start, is_y);
    int count = 0;
    for (int row = start; row < end; ++row) {
        int2 span = make_int2(full0, full1);
        if (e.precise) {
            const float2 high = line_intersection(e, row + 1, is_y);
            span = strip_span(e, row, is_y, low, high);
            low = high;
        }
        f(row, span.x, span.y);
        count += max(0, span.y - span.x);
    }
    return count;
}

// Compact footprint for later passes over grids of at most 256 x 256 tiles
// (32 bytes): (cx, cy, a, b), (c, level or -1 when not precise, det, bounds
// x0 | y0 << 8 | (x1 - 1) << 16 | (y1 - 1) << 24).  unpack_ellipse recomputes
// the extents with the same operations as footprint(), so strips are
// identical.
GS3D_DEV void pack_ellipse(const Ellipse& e, float4& p0, float4& p1) {
    const uint32_t b = (uint32_t)(e.bounds.x & 255) | ((uint32_t)(e.bounds.y & 255) << 8) |
                       ((uint32_t)((e.bounds.z - 1) & 255) << 16) | ((uint32_t)((e.bounds.w - 1) & 255) << 24);
    p0 = make_float4(e.cx, e.cy, e.a, e.b);
    p1 = make_float4(e.c, e.precise ? e.level : -1.0f, e.det, __uint_as_float(b));
}

GS3D_DEV Ellipse unpack_ellipse(float4 p0, float4 p1) {
    Ellipse e;
    e.cx = p0.x;
    e.cy = p0.y;
    e.a = p0.z;
    e.b = p0.w;
    e.c = p1.x;
    e.det = p1.z;
    const uint32_t b = __float_as_uint(p1.w);
    e.bounds = make_int4((int)(b & 255u), (int)((b >> 8) & 255u), (int)((b >> 16) & 255u) + 1, (int)(b >> 24) + 1);
    e.precise = p1.y >= 0.0f;
    e.level = e.precise ? p1.y : 0.0f;
    e.ex = e.ey = 0.0f;
    if (e.precise) {
        e.ex = __builtin_sqrtf(e.level * e.c / e.det);
        e.ey = __builtin_sqrtf(e.level * e.a / e.det);
    }
    return e;
}

// Tiles listed for one projected Gaussian (the count the projection writes,
// projection.py:150-161).
GS3D_DEV int footprint_tiles(float2 center, float4 conic, int radius, int gx, int gy, int mode) {
    if (mode == GS3D_TILE_RADIUS) {
        const int4 r = tile_rect(center.x, center.y, radius, gx, gy);
        return max(0, r.z - r.x) * max(0, r.w - r.y);
    }
    const Ellipse e = footprint(center, conic, radius, gx, gy);
    if (mode == GS3D_TILE_SNUGBOX) return max(0, e.bounds.z - e.bounds.x) * max(0, e.bounds.w - e.bounds.y);
    bool is_y;
    return accutile_strips(e, is_y, [](int, int, int) {});
}

}  // namespace gs3d
