/*
 * bh_oracle.c — CPU restatement of Brush's tile rasterizer (forward and
 * backward).  TEST INFRASTRUCTURE ONLY: the parity checker for the gfx950
 * kernels and the CPU baseline timed by bench.py.  The product never links it.
 *
 * All arithmetic is f32 in the reference's written order; build with
 * -ffp-contract=off (oracle/Makefile).  Citations are to the reference tree
 * (paths relative to crates/).
 */
#include "bh_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "../brush_amd/csrc/bh_math.h"

#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void or_set_threads(int n) { g_threads = n < 1 ? 1 : n; }

void or_expf(const float* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = bh_expf(in[i]);
}

/* the splat Gaussian in base 2 (bh_math.h), for its pins */
void or_exp2_neg(const float* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = bh_exp2_neg(in[i]);
}

void or_power_log2(const float* c00, const float* c01, const float* c11, const float* dx, const float* dy,
                   float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) {
        float a, b, c;
        bh_conic_log2(c00[i], c01[i], c11[i], &a, &b, &c);
        out[i] = bh_power_log2(a, b, c, dx[i], dy[i]);
    }
}

/* The tile walks' quotient (brush_amd/csrc/bh_tile_walk.h div_by_recip):
 * RN(num / den) from y = RN(1 / den) as q0 = RN(num y), r = fma(-den, q0, num),
 * RN(fma(r, y, q0)), for the test that pins it against the division. */
void or_div_by_recip(const float* num, const float* den, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) {
        const float y = 1.0f / den[i];
        const float q0 = num[i] * y;
        const float r = fmaf(-den[i], q0, num[i]);
        out[i] = fmaf(r, y, q0);
    }
}

void or_logf(const float* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = bh_logf(in[i]);
}

int or_get_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* Small linear algebra (brush-cube/src/lib.rs:34-543).                      */
/* ------------------------------------------------------------------------ */

typedef struct { float x, y, z; } v3;
typedef struct { float x, y; } v2;
typedef struct { float w, x, y, z; } qt;
/* column-major: cI_R = column I, row R */
typedef struct { float c0x, c0y, c0z, c1x, c1y, c1z, c2x, c2y, c2z; } m3;
typedef struct { v2 c0, c1, c2; } m23;
typedef struct { float c00, c01, c11; } s2;
typedef struct { float c00, c01, c02, c11, c12, c22; } s3;

static v3 mk3(float x, float y, float z) { v3 r = {x, y, z}; return r; }
static v2 mk2(float x, float y) { v2 r = {x, y}; return r; }
static v3 add3(v3 a, v3 b) { return mk3(a.x + b.x, a.y + b.y, a.z + b.z); }
static v3 sub3(v3 a, v3 b) { return mk3(a.x - b.x, a.y - b.y, a.z - b.z); }
static v3 scl3(v3 a, float s) { return mk3(a.x * s, a.y * s, a.z * s); }
static float dot3(v3 a, v3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
static float len3(v3 a) { return sqrtf(dot3(a, a)); }
static int fin3(v3 a) { return bh_is_finite(a.x) && bh_is_finite(a.y) && bh_is_finite(a.z); }
static v2 add2(v2 a, v2 b) { return mk2(a.x + b.x, a.y + b.y); }
static v2 scl2(v2 a, float s) { return mk2(a.x * s, a.y * s); }
static float dot2(v2 a, v2 b) { return a.x * b.x + a.y * b.y; }

static float qdot(qt a, qt b) { return a.w * b.w + a.x * b.x + a.y * b.y + a.z * b.z; }
static qt qscale(qt a, float s) { qt r = {a.w * s, a.x * s, a.y * s, a.z * s}; return r; }
/* Quat::normalize (lib.rs:185-188) */
static qt qnormalize(qt q) { return qscale(q, 1.0f / sqrtf(qdot(q, q))); }
/* Quat::to_mat3 (lib.rs:190-216) */
static m3 qmat(qt q) {
    float x2 = q.x * q.x, y2 = q.y * q.y, z2 = q.z * q.z;
    float xy = q.x * q.y, xz = q.x * q.z, yz = q.y * q.z;
    float wx = q.w * q.x, wy = q.w * q.y, wz = q.w * q.z;
    m3 m;
    m.c0x = 1.0f - 2.0f * (y2 + z2);
    m.c0y = 2.0f * (xy + wz);
    m.c0z = 2.0f * (xz - wy);
    m.c1x = 2.0f * (xy - wz);
    m.c1y = 1.0f - 2.0f * (x2 + z2);
    m.c1z = 2.0f * (yz + wx);
    m.c2x = 2.0f * (xz + wy);
    m.c2y = 2.0f * (yz - wx);
    m.c2z = 1.0f - 2.0f * (x2 + y2);
    return m;
}
static v3 col0(m3 m) { return mk3(m.c0x, m.c0y, m.c0z); }
static v3 col1(m3 m) { return mk3(m.c1x, m.c1y, m.c1z); }
static v3 col2(m3 m) { return mk3(m.c2x, m.c2y, m.c2z); }
static v3 row0(m3 m) { return mk3(m.c0x, m.c1x, m.c2x); }
static v3 row1(m3 m) { return mk3(m.c0y, m.c1y, m.c2y); }
static v3 row2(m3 m) { return mk3(m.c0z, m.c1z, m.c2z); }
static m3 from_cols(v3 a, v3 b, v3 c) {
    m3 m = {a.x, a.y, a.z, b.x, b.y, b.z, c.x, c.y, c.z};
    return m;
}
/* Mat3::mul_vec3 (lib.rs:262-268): col0*x + col1*y + col2*z */
static v3 m3mulv(m3 m, v3 v) { return add3(add3(scl3(col0(m), v.x), scl3(col1(m), v.y)), scl3(col2(m), v.z)); }
/* Mat3::transpose_mul_vec3 (lib.rs:270-273) */
static v3 m3tmulv(m3 m, v3 v) { return mk3(dot3(col0(m), v), dot3(col1(m), v), dot3(col2(m), v)); }
/* Mat3::mul_mat3 (lib.rs:275-282) */
static m3 m3mul(m3 a, m3 b) { return from_cols(m3mulv(a, col0(b)), m3mulv(a, col1(b)), m3mulv(a, col2(b))); }
/* Mat3::mul_diag (lib.rs:284-291) */
static m3 m3diag(m3 m, v3 s) { return from_cols(scl3(col0(m), s.x), scl3(col1(m), s.y), scl3(col2(m), s.z)); }
/* Mat3::outer_product_self (lib.rs:305-318) */
static s3 m3outer(m3 m) {
    v3 r0 = row0(m), r1 = row1(m), r2 = row2(m);
    s3 s = {dot3(r0, r0), dot3(r0, r1), dot3(r0, r2), dot3(r1, r1), dot3(r1, r2), dot3(r2, r2)};
    return s;
}
/* Mat2x3::mul_vec3 (lib.rs:341-347) */
static v2 m23mulv(m23 m, v3 v) { return add2(add2(scl2(m.c0, v.x), scl2(m.c1, v.y)), scl2(m.c2, v.z)); }
/* Mat2x3::mul_mat3 (lib.rs:332-339) */
static m23 m23mul(m23 m, m3 n) {
    m23 r = {m23mulv(m, col0(n)), m23mulv(m, col1(n)), m23mulv(m, col2(n))};
    return r;
}
static v3 m23row0(m23 m) { return mk3(m.c0.x, m.c1.x, m.c2.x); }
static v3 m23row1(m23 m) { return mk3(m.c0.y, m.c1.y, m.c2.y); }
/* Mat2x3::gram_matrix (lib.rs:377-383) */
static s2 m23gram(m23 m) {
    s2 s;
    s.c00 = m.c0.x * m.c0.x + m.c1.x * m.c1.x + m.c2.x * m.c2.x;
    s.c01 = m.c0.x * m.c0.y + m.c1.x * m.c1.y + m.c2.x * m.c2.y;
    s.c11 = m.c0.y * m.c0.y + m.c1.y * m.c1.y + m.c2.y * m.c2.y;
    return s;
}
/* Sym2::mul_vec2 (lib.rs:405-408) */
static v2 s2mulv(s2 s, v2 v) { return add2(scl2(mk2(s.c00, s.c01), v.x), scl2(mk2(s.c01, s.c11), v.y)); }
/* Sym2::mul_mat2x3 (lib.rs:425-432) */
static m23 s2mulm23(s2 s, m23 n) {
    m23 r = {s2mulv(s, n.c0), s2mulv(s, n.c1), s2mulv(s, n.c2)};
    return r;
}
/* Mat2x3::transpose_congruence_sym2 (lib.rs:357-370) */
static s3 m23tcong(m23 m, s2 s) {
    v2 sc0 = s2mulv(s, m.c0), sc1 = s2mulv(s, m.c1), sc2 = s2mulv(s, m.c2);
    s3 r = {dot2(m.c0, sc0), dot2(m.c0, sc1), dot2(m.c0, sc2), dot2(m.c1, sc1), dot2(m.c1, sc2), dot2(m.c2, sc2)};
    return r;
}
static s2 s2scale(s2 s, float f) { s2 r = {s.c00 * f, s.c01 * f, s.c11 * f}; return r; }
static float s2maxabs(s2 s) { return bh_maxf(bh_maxf(bh_absf(s.c00), bh_absf(s.c11)), bh_absf(s.c01)); }
/* Sym2::inverse (lib.rs:434-445) */
static s2 s2inv(s2 s) {
    float det = s.c00 * s.c11 - s.c01 * s.c01;
    int inv = det > 0.0f;
    float inv_det = inv ? 1.0f / det : 0.0f;
    s2 r = {s.c11 * inv_det, -s.c01 * inv_det, s.c00 * inv_det};
    return r;
}
/* Sym2::det2_strict (lib.rs:447-453) */
static float s2det(s2 s) {
    float ad = s.c00 * s.c11;
    float bc = s.c01 * s.c01;
    return ad - bc;
}
static int s2fin(s2 s) { return bh_is_finite(s.c00) && bh_is_finite(s.c11) && bh_is_finite(s.c01); }
/* Sym3 rows and products (lib.rs:472-543) */
static v3 s3row0(s3 s) { return mk3(s.c00, s.c01, s.c02); }
static v3 s3row1(s3 s) { return mk3(s.c01, s.c11, s.c12); }
static v3 s3row2(s3 s) { return mk3(s.c02, s.c12, s.c22); }
static v3 s3mulv(s3 s, v3 v) { return add3(add3(scl3(s3row0(s), v.x), scl3(s3row1(s), v.y)), scl3(s3row2(s), v.z)); }
static s3 s3scale(s3 s, float f) { s3 r = {s.c00 * f, s.c01 * f, s.c02 * f, s.c11 * f, s.c12 * f, s.c22 * f}; return r; }
static m3 s3mulm3(s3 s, m3 m) { return from_cols(s3mulv(s, col0(m)), s3mulv(s, col1(m)), s3mulv(s, col2(m))); }
static s3 s3cong(s3 s, m3 m) {
    v3 sr0 = s3mulv(s, row0(m)), sr1 = s3mulv(s, row1(m)), sr2 = s3mulv(s, row2(m));
    s3 r = {dot3(row0(m), sr0), dot3(row0(m), sr1), dot3(row0(m), sr2), dot3(row1(m), sr1), dot3(row1(m), sr2), dot3(row2(m), sr2)};
    return r;
}
static s3 s3tcong(s3 s, m3 m) {
    v3 sc0 = s3mulv(s, col0(m)), sc1 = s3mulv(s, col1(m)), sc2 = s3mulv(s, col2(m));
    s3 r = {dot3(col0(m), sc0), dot3(col0(m), sc1), dot3(col0(m), sc2), dot3(col1(m), sc1), dot3(col1(m), sc2), dot3(col2(m), sc2)};
    return r;
}

/* ------------------------------------------------------------------------ */
/* Camera / projection helpers                                               */
/* ------------------------------------------------------------------------ */

static m3 view_rot(const bh_project_uniforms* u) {
    const float* v = u->viewmat;
    m3 m = {v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7], v[8]};
    return m;
}
/* world_to_cam (kernels/helpers.rs:477-482): R*mean + t */
static v3 world_to_cam(const bh_project_uniforms* u, v3 mean) {
    return add3(m3mulv(view_rot(u), mean), mk3(u->viewmat[9], u->viewmat[10], u->viewmat[11]));
}
/* project_pinhole (camera_model/pinhole.rs:24-30) */
static void project_pinhole(const bh_project_uniforms* u, v3 p, float* ox, float* oy) {
    float inv_z = 1.0f / p.z;
    *ox = u->fx * p.x * inv_z + u->cx;
    *oy = u->fy * p.y * inv_z + u->cy;
}
/* calculate_project_jacobian_pinhole (pinhole.rs:32-56) */
static m23 jac_pinhole(const bh_project_uniforms* u, v3 p) {
    float inv_z = 1.0f / p.z;
    float dx = u->fx * inv_z;
    float dy = u->fy * inv_z;
    float cxl = bh_clampf(p.x * inv_z, u->lim_neg_x, u->lim_pos_x);
    float cyl = bh_clampf(p.y * inv_z, u->lim_neg_y, u->lim_pos_y);
    m23 m = {mk2(dx, 0.0f), mk2(0.0f, dy), mk2(-dx * cxl, -dy * cyl)};
    return m;
}
/* ---- camera models (kernels/camera_model/{kannala_brandt_4,
 * radial_tangential_8,thin_prism_fisheye}.rs).  u->camera_params holds the
 * coefficients in the reference's struct order: KB4 k1..k4, RT8 k1..k6 p1 p2,
 * TPF k1..k4 p1 p2 sx1 sy1. */
static m23 mkm23(float a00, float a10, float a01, float a11, float a02, float a12) {
    m23 m = {mk2(a00, a10), mk2(a01, a11), mk2(a02, a12)};
    return m;
}
/* project_kb4 (kannala_brandt_4.rs:18-52) */
static v2 kb4_project(const bh_project_uniforms* u, v3 p) {
    const float* k = u->camera_params;
    float inv_z = 1.0f / p.z;
    float pu = u->fx * p.x * inv_z + u->cx;
    float pv = u->fy * p.y * inv_z + u->cy;
    float r = sqrtf(p.x * p.x + p.y * p.y);
    float th = bh_atan2f(r, p.z);
    float th2 = th * th;
    float th4 = th2 * th2;
    float th6 = th2 * th4;
    float th8 = th4 * th4;
    float d = th * (1.0f + k[0] * th2 + k[1] * th4 + k[2] * th6 + k[3] * th8);
    float inv_r = 1.0f / r;
    float fu = u->fx * (d * p.x * inv_r) + u->cx;
    float fv = u->fy * (d * p.y * inv_r) + u->cy;
    if (r < 1e-6f) return mk2(pu, pv);
    return mk2(fu, fv);
}
/* calculate_project_jacobian_kb4 (kannala_brandt_4.rs:54-136) */
static m23 kb4_jacobian(const bh_project_uniforms* u, v3 p) {
    const float* k = u->camera_params;
    float fx = u->fx, fy = u->fy, x = p.x, y = p.y, z = p.z;
    float inv_z = 1.0f / z;
    float x2 = x * x, y2 = y * y, xy = x * y;
    float r2 = x2 + y2;
    float r = sqrtf(r2);
    float inv_r = 1.0f / r;
    float inv_r3 = inv_r * inv_r * inv_r;
    float rho2 = r2 + z * z;
    float inv_rho2 = 1.0f / rho2;
    float inv_rho2_r = inv_rho2 * inv_r;
    float th = bh_atan2f(r, z);
    float th2 = th * th, th4 = th2 * th2, th6 = th4 * th2, th8 = th4 * th4;
    float d = th * (1.0f + k[0] * th2 + k[1] * th4 + k[2] * th6 + k[3] * th8);
    float ddt = 1.0f + 3.0f * k[0] * th2 + 5.0f * k[1] * th4 + 7.0f * k[2] * th6 + 9.0f * k[3] * th8;
    float dth_dx = x * z * inv_rho2_r;
    float dth_dy = y * z * inv_rho2_r;
    float dth_dz = -r * inv_rho2;
    float dd_dx = ddt * dth_dx, dd_dy = ddt * dth_dy, dd_dz = ddt * dth_dz;
    float xr = x * inv_r;
    float dxr_dx = y2 * inv_r3;
    float dxr_dy = -xy * inv_r3;
    float yr = y * inv_r;
    float dyr_dx = -xy * inv_r3;
    float dyr_dy = x2 * inv_r3;
    if (r < 1e-6f) {
        float ddx = fx * inv_z, ddy = fy * inv_z;
        return mkm23(ddx, 0.0f, 0.0f, ddy, -ddx * x * inv_z, -ddy * y * inv_z);
    }
    return mkm23(fx * (dd_dx * xr + d * dxr_dx), fy * (dd_dx * yr + d * dyr_dx), fx * (dd_dy * xr + d * dxr_dy),
                 fy * (dd_dy * yr + d * dyr_dy), fx * (dd_dz * xr), fy * (dd_dz * yr));
}
/* project_rt8 (radial_tangential_8.rs:24-69) */
static v2 rt8_project(const bh_project_uniforms* u, v3 p) {
    const float* k = u->camera_params;
    float p1 = k[6], p2 = k[7];
    float xn = p.x / p.z, yn = p.y / p.z;
    float xn2 = xn * xn, yn2 = yn * yn;
    float r2 = xn2 + yn2;
    float r4 = r2 * r2;
    float r6 = r4 * r2;
    float d = (1.0f + k[0] * r2 + k[1] * r4 + k[2] * r6) / (1.0f + k[3] * r2 + k[4] * r4 + k[5] * r6);
    float xy = xn * yn;
    float xd = xn * d + 2.0f * p1 * xy + p2 * (r2 + 2.0f * xn2);
    float yd = yn * d + 2.0f * p2 * xy + p1 * (r2 + 2.0f * yn2);
    return mk2(u->fx * xd + u->cx, u->fy * yd + u->cy);
}
/* radial term R(r2) = N/Dn and R', R'' with respect to r2 (both RT8 paths) */
typedef struct { float n, dn, np, dnp; } rt8_polys;
/* calculate_project_jacobian_rt8 (radial_tangential_8.rs:71-146) */
static m23 rt8_jacobian(const bh_project_uniforms* u, v3 p) {
    const float* k = u->camera_params;
    float p1 = k[6], p2 = k[7], fx = u->fx, fy = u->fy, z = p.z;
    float inv_z = 1.0f / z;
    float inv_z2 = inv_z * inv_z;
    float xn = bh_clampf(p.x * inv_z, u->lim_neg_x, u->lim_pos_x);
    float yn = bh_clampf(p.y * inv_z, u->lim_neg_y, u->lim_pos_y);
    float xc = xn * z, yc = yn * z;
    float r2 = xn * xn + yn * yn;
    float r4 = r2 * r2;
    float r6 = r4 * r2;
    float n = 1.0f + k[0] * r2 + k[1] * r4 + k[2] * r6;
    float dn = 1.0f + k[3] * r2 + k[4] * r4 + k[5] * r6;
    float np = k[0] + 2.0f * k[1] * r2 + 3.0f * k[2] * r4;
    float dnp = k[3] + 2.0f * k[4] * r2 + 3.0f * k[5] * r4;
    float inv_dn = 1.0f / dn;
    float inv_dn2 = inv_dn * inv_dn;
    float rv = n * inv_dn;
    float rp = (np * dn - n * dnp) * inv_dn2;
    float d00 = rv + 2.0f * xn * xn * rp + 2.0f * p1 * yn + 6.0f * p2 * xn;
    float d01 = 2.0f * xn * yn * rp + 2.0f * p1 * xn + 2.0f * p2 * yn;
    float d10 = d01;
    float d11 = rv + 2.0f * yn * yn * rp + 6.0f * p1 * yn + 2.0f * p2 * xn;
    return mkm23(fx * d00 * inv_z, fy * d10 * inv_z, fx * d01 * inv_z, fy * d11 * inv_z,
                 -fx * (d00 * xc + d01 * yc) * inv_z2, -fy * (d10 * xc + d11 * yc) * inv_z2);
}
/* thin_prism_polys (thin_prism_fisheye.rs:37-63): out = Nu, Nv, dNu/dx,
 * dNu/dy, dNv/dx, dNv/dy at camera-space (x, y) */
static void tpf_polys(const bh_project_uniforms* u, float x, float y, float* o) {
    float p1 = u->camera_params[4], p2 = u->camera_params[5];
    float sx1 = u->camera_params[6], sy1 = u->camera_params[7];
    float x2 = x * x, y2 = y * y, xy = x * y;
    float r2 = x2 + y2;
    o[0] = 2.0f * p1 * xy + p2 * (3.0f * x2 + y2) + sx1 * r2;
    o[1] = 2.0f * p2 * xy + p1 * (x2 + 3.0f * y2) + sy1 * r2;
    o[2] = 2.0f * (p1 * y + (3.0f * p2 + sx1) * x);
    o[3] = 2.0f * (p1 * x + (p2 + sx1) * y);
    o[4] = 2.0f * (p2 * y + (p1 + sy1) * x);
    o[5] = 2.0f * (p2 * x + (3.0f * p1 + sy1) * y);
}
/* project_tpf (thin_prism_fisheye.rs:65-81) */
static v2 tpf_project(const bh_project_uniforms* u, v3 p) {
    v2 kb = kb4_project(u, p);
    float inv_z = 1.0f / p.z;
    float inv_z2 = inv_z * inv_z;
    float t[6];
    tpf_polys(u, p.x, p.y, t);
    return mk2(kb.x + u->fx * t[0] * inv_z2, kb.y + u->fy * t[1] * inv_z2);
}
/* calculate_project_jacobian_tpf (thin_prism_fisheye.rs:83-114) */
static m23 tpf_jacobian(const bh_project_uniforms* u, v3 p) {
    m23 kb = kb4_jacobian(u, p);
    float fx = u->fx, fy = u->fy;
    float inv_z = 1.0f / p.z;
    float inv_z2 = inv_z * inv_z;
    float inv_z3 = inv_z2 * inv_z;
    float t[6];
    tpf_polys(u, p.x, p.y, t);
    return mkm23(kb.c0.x + fx * t[2] * inv_z2, kb.c0.y + fy * t[4] * inv_z2, kb.c1.x + fx * t[3] * inv_z2,
                 kb.c1.y + fy * t[5] * inv_z2, kb.c2.x + -2.0f * fx * t[0] * inv_z3,
                 kb.c2.y + -2.0f * fy * t[1] * inv_z3);
}
/* project (camera_model/mod.rs:50-62) */
static void project_point(const bh_project_uniforms* u, v3 p, float* ox, float* oy) {
    v2 r;
    switch (u->camera_model) {
        case BH_CAMERA_KB4: r = kb4_project(u, p); break;
        case BH_CAMERA_RT8: r = rt8_project(u, p); break;
        case BH_CAMERA_TPF: r = tpf_project(u, p); break;
        default: project_pinhole(u, p, ox, oy); return;
    }
    *ox = r.x;
    *oy = r.y;
}
/* calculate_project_jacobian (camera_model/mod.rs:64-80) */
static m23 cam_jacobian(const bh_project_uniforms* u, v3 p) {
    switch (u->camera_model) {
        case BH_CAMERA_KB4: return kb4_jacobian(u, p);
        case BH_CAMERA_RT8: return rt8_jacobian(u, p);
        case BH_CAMERA_TPF: return tpf_jacobian(u, p);
        default: return jac_pinhole(u, p);
    }
}
/* the depth cull of project_forward (project_forward.rs:49-62) */
static int depth_culled(const bh_project_uniforms* u, v3 mean_c) {
    if (u->camera_model == BH_CAMERA_PINHOLE) return mean_c.z < 0.01f;
    float r = sqrtf(mean_c.x * mean_c.x + mean_c.y * mean_c.y);
    return bh_atan2f(r, mean_c.z) > u->half_max_render_fov;
}
/* calc_cov2d (kernels/helpers.rs:297-330) */
static s2 calc_cov2d(const bh_project_uniforms* u, v3 scale, qt quat, v3 mean_c) {
    m3 ns = m3diag(m3mul(view_rot(u), qmat(quat)), scale);
    m23 jac = cam_jacobian(u, mean_c);
    m23 v = m23mul(jac, ns);
    s2 raw = m23gram(v);
    float lim = 1.0e18f;
    float max_abs = s2maxabs(raw);
    float scale_down = max_abs > lim ? lim / max_abs : 1.0f;
    return s2scale(raw, scale_down);
}
/* compensate_cov2d (kernels/helpers.rs:332-350) */
static s2 compensate_cov2d(s2 c, uint32_t mip, float* comp) {
    float blur = mip ? 0.1f : 0.3f;
    s2 b = {c.c00 + blur, c.c01, c.c11 + blur};
    float fc = 1.0f;
    if (mip) {
        float det_raw = bh_maxf(s2det(c), 0.0f);
        float det_b = s2det(b);
        fc = sqrtf(det_raw / det_b);
    }
    *comp = fc;
    return b;
}
/* compute_bbox_extent (kernels/helpers.rs:227-241) */
static void bbox_extent(s2 conic, float pt, float* ex, float* ey) {
    float det = conic.c00 * conic.c11 - conic.c01 * conic.c01;
    int degenerate = det <= 0.0f;
    float inv_det = degenerate ? 0.0f : 1.0f / det;
    float x = sqrtf(2.0f * pt * conic.c11 * inv_det);
    float y = sqrtf(2.0f * pt * conic.c00 * inv_det);
    *ex = degenerate ? -1.0f : x;
    *ey = degenerate ? -1.0f : y;
}
typedef struct { uint32_t min_x, min_y, max_x, max_y; } tbox;
/* get_bbox / get_tile_bbox (kernels/helpers.rs:260-295) */
static tbox tile_bbox(float mx, float my, float ex, float ey, uint32_t bw, uint32_t bh, uint32_t th) {
    float cx = mx / 16.0f, cy = my / (float)th, dx = ex / 16.0f, dy = ey / (float)th;
    float bwf = (float)bw, bhf = (float)bh;
    tbox b;
    b.min_x = (uint32_t)bh_clampf(cx - dx, 0.0f, bwf);
    b.min_y = (uint32_t)bh_clampf(cy - dy, 0.0f, bhf);
    b.max_x = (uint32_t)bh_clampf(cx + dx + 1.0f, 0.0f, bwf);
    b.max_y = (uint32_t)bh_clampf(cy + dy + 1.0f, 0.0f, bhf);
    return b;
}
/* calc_sigma (brush-cube/src/lib.rs:632-638) */
static float calc_sigma(float px, float py, s2 c, float x, float y) {
    float dx = px - x;
    float dy = py - y;
    return 0.5f * (c.c00 * dx * dx + c.c11 * dy * dy) + c.c01 * dx * dy;
}
/* will_primitive_contribute (kernels/helpers.rs:385-424), 16x16 tile rect */
static int will_contribute(uint32_t tx, uint32_t ty, uint32_t th, float mx, float my, s2 c, float pt) {
    float min_x = (float)(tx * 16u), min_y = (float)(ty * th);
    float max_x = min_x + 16.0f, max_y = min_y + (float)th;
    int x_left = mx < min_x, x_right = mx > max_x;
    int in_x = !(x_left || x_right);
    int y_above = my < min_y, y_below = my > max_y;
    int in_y = !(y_above || y_below);
    int hit = in_x && in_y;
    if (!hit) {
        float corner_x = x_left ? min_x : max_x;
        float corner_y = y_above ? min_y : max_y;
        float width = max_x - min_x;
        float height = max_y - min_y;
        float dxf = x_left ? width : -width;
        float dyf = y_above ? height : -height;
        float diff_x = mx - corner_x;
        float diff_y = my - corner_y;
        float tx_raw = (dxf * c.c00 * diff_x + dxf * c.c01 * diff_y) / (dxf * c.c00 * dxf);
        float ty_raw = (dyf * c.c01 * diff_x + dyf * c.c11 * diff_y) / (dyf * c.c11 * dyf);
        float tt_x = in_y ? 0.0f : bh_clampf(tx_raw, 0.0f, 1.0f);
        float tt_y = in_x ? 0.0f : bh_clampf(ty_raw, 0.0f, 1.0f);
        float px = corner_x + tt_x * dxf;
        float py = corner_y + tt_y * dyf;
        hit = calc_sigma(px, py, c, mx, my) <= pt;
    }
    return hit;
}

/* ------------------------------------------------------------------------ */
/* project_forward (kernels/project_forward.rs:20-144)                       */
/* Pinned by: fuzz cull cases (bench-test/tests/fuzz.rs:330-490), brute      */
/* force tile enumeration, and the gsplat goldens through the full forward.  */
/* ------------------------------------------------------------------------ */

/* Returns 1 and fills outputs if the splat survives culling. */
static int project_one(const bh_project_uniforms* u, const float* t, float raw_opac, uint32_t mip, uint32_t th,
                       uint32_t* count, float* radius, float* depth) {
    v3 mean_c = world_to_cam(u, mk3(t[0], t[1], t[2]));
    if (!(fin3(mean_c) && mean_c.z <= 1.0e10f)) return 0;
    if (depth_culled(u, mean_c)) return 0;
    v3 scale = mk3(bh_expf(t[7]), bh_expf(t[8]), bh_expf(t[9]));
    if (!fin3(scale)) return 0;
    qt qu = {t[3], t[4], t[5], t[6]};
    float qn = qdot(qu, qu);
    if (!(qn >= 1.0e-6f && bh_is_finite(qn))) return 0;
    if (!bh_is_finite(raw_opac)) return 0;
    qt q = qnormalize(qu);
    s2 raw_cov = calc_cov2d(u, scale, q, mean_c);
    float comp;
    s2 cov = compensate_cov2d(raw_cov, mip, &comp);
    float opac = bh_sigmoidf(raw_opac) * comp;
    if (!s2fin(cov)) return 0;
    float mx, my;
    project_point(u, mean_c, &mx, &my);
    if (!(opac >= 1.0f / 255.0f)) return 0;
    float pt = bh_logf(opac * 255.0f);
    s2 conic = s2inv(cov);
    float ex, ey;
    bbox_extent(conic, pt, &ex, &ey);
    if (!(ex >= 0.0f && ey >= 0.0f)) return 0;
    float wf = (float)u->img_w, hf = (float)u->img_h;
    int on_screen = mx + ex > 0.0f && mx - ex < wf && my + ey > 0.0f && my - ey < hf;
    if (!on_screen) return 0;
    tbox bb = tile_bbox(mx, my, ex, ey, u->tile_bw, u->tile_bh, th);
    uint32_t hits = 0;
    for (uint32_t ty = bb.min_y; ty < bb.max_y; ty++)
        for (uint32_t tx = bb.min_x; tx < bb.max_x; tx++)
            if (will_contribute(tx, ty, th, mx, my, conic, pt)) hits++;
    *count = hits;
    *radius = bh_maxf(ex / wf, ey / hf);
    *depth = mean_c.z;
    return 1;
}

uint64_t or_project_forward(const bh_project_uniforms* u, const float* transforms,
                            const float* raw_opac, uint32_t n, uint32_t mip, uint32_t tile_h,
                            uint32_t* intersect_counts, float* max_radius, float* depths,
                            uint8_t* visible_mask) {
    uint64_t total = 0;
#pragma omp parallel for schedule(dynamic, 4096) reduction(+ : total) num_threads(g_threads)
    for (int64_t i = 0; i < (int64_t)n; i++) {
        uint32_t c = 0;
        float r = 0.0f, d = 0.0f;
        int vis = project_one(u, transforms + (size_t)i * 10, raw_opac[i], mip, tile_h, &c, &r, &d);
        intersect_counts[i] = vis ? c : 0u;
        max_radius[i] = vis ? r : 0.0f;
        depths[i] = vis ? d : 0.0f;
        visible_mask[i] = (uint8_t)vis;
        total += vis ? c : 0u;
    }
    return total;
}

/* ------------------------------------------------------------------------ */
/* Stable sort: textbook bottom-up merge sort on (key & mask, value) pairs.  */
/* Semantics of brush-sort radix_argsort (brush-sort/src/lib.rs:16-129): a   */
/* stable ascending sort on the low `sorting_bits` key bits; the returned    */
/* keys are the original keys.  Pinned by stability/permutation tests.       */
/* ------------------------------------------------------------------------ */

void or_stable_sort(uint32_t* keys, uint32_t* vals, uint64_t n, uint32_t sorting_bits) {
    if (n < 2) return;
    uint32_t mask = sorting_bits >= 32 ? 0xFFFFFFFFu : ((1u << sorting_bits) - 1u);
    uint32_t* k2 = (uint32_t*)malloc(n * sizeof(uint32_t));
    uint32_t* v2b = (uint32_t*)malloc(n * sizeof(uint32_t));
    uint32_t *sk = keys, *sv = vals, *dk = k2, *dv = v2b;
    for (uint64_t w = 1; w < n; w *= 2) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
        for (int64_t lo = 0; lo < (int64_t)n; lo += (int64_t)(2 * w)) {
            uint64_t mid = (uint64_t)lo + w < n ? (uint64_t)lo + w : n;
            uint64_t hi = (uint64_t)lo + 2 * w < n ? (uint64_t)lo + 2 * w : n;
            uint64_t i = (uint64_t)lo, j = mid, o = (uint64_t)lo;
            while (i < mid && j < hi) {
                if ((sk[j] & mask) < (sk[i] & mask)) {
                    dk[o] = sk[j]; dv[o] = sv[j]; j++;
                } else {
                    dk[o] = sk[i]; dv[o] = sv[i]; i++;
                }
                o++;
            }
            while (i < mid) { dk[o] = sk[i]; dv[o] = sv[i]; i++; o++; }
            while (j < hi) { dk[o] = sk[j]; dv[o] = sv[j]; j++; o++; }
        }
        uint32_t* t;
        t = sk; sk = dk; dk = t;
        t = sv; sv = dv; dv = t;
    }
    if (sk != keys) {
        memcpy(keys, sk, n * sizeof(uint32_t));
        memcpy(vals, sv, n * sizeof(uint32_t));
    }
    free(k2);
    free(v2b);
}

/* Inclusive scan (brush-prefix-sum/src/lib.rs:11-87). Closed form. */
void or_prefix_sum(const uint32_t* in, uint32_t* out, uint64_t n) {
    uint32_t acc = 0;
    for (uint64_t i = 0; i < n; i++) {
        acc += in[i];
        out[i] = acc;
    }
}

/* ------------------------------------------------------------------------ */
/* SH -> RGB (kernels/sh.rs:157-247). Coefficient k of channel ch is at      */
/* base + 3k + ch.                                                           */
/* ------------------------------------------------------------------------ */
static v3 rd3(const float* c, uint32_t k) { return mk3(c[3 * k], c[3 * k + 1], c[3 * k + 2]); }

static v3 sh_to_color(const float* c, uint32_t deg, v3 v) {
    v3 color = scl3(rd3(c, 0), 0.2820948f);
    if (deg >= 1) {
        float f0a = 0.4886025f;
        color = add3(color, scl3(rd3(c, 1), -f0a * v.y));
        color = add3(color, scl3(rd3(c, 2), f0a * v.z));
        color = add3(color, scl3(rd3(c, 3), -f0a * v.x));
        if (deg >= 2) {
            float z2 = v.z * v.z;
            float f0b = -1.0925485f * v.z;
            float f1a = 0.54627424f;
            float fc1 = v.x * v.x - v.y * v.y;
            float fs1 = 2.0f * v.x * v.y;
            float p4 = f1a * fs1, p5 = f0b * v.y, p6 = 0.9461747f * z2 - 0.31539157f;
            float p7 = f0b * v.x, p8 = f1a * fc1;
            color = add3(color, scl3(rd3(c, 4), p4));
            color = add3(color, scl3(rd3(c, 5), p5));
            color = add3(color, scl3(rd3(c, 6), p6));
            color = add3(color, scl3(rd3(c, 7), p7));
            color = add3(color, scl3(rd3(c, 8), p8));
            if (deg >= 3) {
                float f0c = -2.285229f * z2 + 0.4570458f;
                float f1b = 1.4453057f * v.z;
                float f2a = -0.5900436f;
                float fc2 = v.x * fc1 - v.y * fs1;
                float fs2 = v.x * fs1 + v.y * fc1;
                float p12 = v.z * (1.8658817f * z2 - 1.119529f);
                float p9 = f2a * fs2, p10 = f1b * fs1, p11 = f0c * v.y;
                float p13 = f0c * v.x, p14 = f1b * fc1, p15 = f2a * fc2;
                color = add3(color, scl3(rd3(c, 9), p9));
                color = add3(color, scl3(rd3(c, 10), p10));
                color = add3(color, scl3(rd3(c, 11), p11));
                color = add3(color, scl3(rd3(c, 12), p12));
                color = add3(color, scl3(rd3(c, 13), p13));
                color = add3(color, scl3(rd3(c, 14), p14));
                color = add3(color, scl3(rd3(c, 15), p15));
                if (deg >= 4) {
                    float f0d = v.z * (-4.683326f * z2 + 2.0071396f);
                    float f1c = 3.3116114f * z2 - 0.47308735f;
                    float f2b = -1.7701308f * v.z;
                    float f3a = 0.62583575f;
                    float fc3 = v.x * fc2 - v.y * fs2;
                    float fs3 = v.x * fs2 + v.y * fc2;
                    float p20 = 1.9843135f * v.z * p12 - 1.0062306f * p6;
                    float p16 = f3a * fs3, p17 = f2b * fs2, p18 = f1c * fs1, p19 = f0d * v.y;
                    float p21 = f0d * v.x, p22 = f1c * fc1, p23 = f2b * fc2, p24 = f3a * fc3;
                    color = add3(color, scl3(rd3(c, 16), p16));
                    color = add3(color, scl3(rd3(c, 17), p17));
                    color = add3(color, scl3(rd3(c, 18), p18));
                    color = add3(color, scl3(rd3(c, 19), p19));
                    color = add3(color, scl3(rd3(c, 20), p20));
                    color = add3(color, scl3(rd3(c, 21), p21));
                    color = add3(color, scl3(rd3(c, 22), p22));
                    color = add3(color, scl3(rd3(c, 23), p23));
                    color = add3(color, scl3(rd3(c, 24), p24));
                }
            }
        }
    }
    return color;
}

/* ------------------------------------------------------------------------ */
/* project_visible (kernels/project_visible.rs:22-89)                        */
/* ------------------------------------------------------------------------ */
void or_project_visible(const bh_project_uniforms* u, const float* transforms,
                        const float* sh_coeffs, const float* raw_opac,
                        const uint32_t* global_from_compact_gid, uint32_t num_visible,
                        uint32_t sh_degree, uint32_t mip, float* projected) {
    uint32_t nc = (sh_degree + 1) * (sh_degree + 1);
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int64_t ci = 0; ci < (int64_t)num_visible; ci++) {
        uint32_t g = global_from_compact_gid[ci];
        const float* t = transforms + (size_t)g * 10;
        v3 mean = mk3(t[0], t[1], t[2]);
        v3 scale = mk3(bh_expf(t[7]), bh_expf(t[8]), bh_expf(t[9]));
        qt qu = {t[3], t[4], t[5], t[6]};
        qt q = qnormalize(qu);
        v3 mean_c = world_to_cam(u, mean);
        s2 raw_cov = calc_cov2d(u, scale, q, mean_c);
        float comp;
        s2 cov = compensate_cov2d(raw_cov, mip, &comp);
        float opac = bh_sigmoidf(raw_opac[g]) * comp;
        s2 conic = s2inv(cov);
        float mx, my;
        project_point(u, mean_c, &mx, &my);
        v3 v = sub3(mean, mk3(u->camera_pos[0], u->camera_pos[1], u->camera_pos[2]));
        v = scl3(v, 1.0f / len3(v));
        v3 raw = sh_to_color(sh_coeffs + (size_t)g * nc * 3, sh_degree, v);
        float cr = raw.x + 0.5f, cg = raw.y + 0.5f, cb = raw.z + 0.5f;
        float* p = projected + (size_t)ci * 10;
        p[0] = mx;
        p[1] = my;
        p[2] = conic.c00;
        p[3] = conic.c01;
        p[4] = conic.c11;
        p[5] = opac;
        p[6] = bh_clampf(bh_is_finite(cr) ? cr : 0.0f, -100.0f, 100.0f);
        p[7] = bh_clampf(bh_is_finite(cg) ? cg : 0.0f, -100.0f, 100.0f);
        p[8] = bh_clampf(bh_is_finite(cb) ? cb : 0.0f, -100.0f, 100.0f);
        p[9] = mean_c.z;
    }
}

/* ------------------------------------------------------------------------ */
/* map_gaussians_to_intersect (kernels/map_gaussians.rs:14-92)               */
/* ------------------------------------------------------------------------ */
void or_map_intersects(uint32_t tile_bw, uint32_t tile_bh, uint32_t tile_h, const float* projected,
                       const uint32_t* cum, uint32_t num_visible,
                       uint32_t* tile_id_from_isect, uint32_t* compact_gid_from_isect) {
#pragma omp parallel for schedule(dynamic, 1024) num_threads(g_threads)
    for (int64_t ci = 0; ci < (int64_t)num_visible; ci++) {
        const float* p = projected + (size_t)ci * 10;
        float mx = p[0], my = p[1];
        s2 conic = {p[2], p[3], p[4]};
        float pt = bh_logf(p[5] * 255.0f);
        float ex, ey;
        bbox_extent(conic, pt, &ex, &ey);
        tbox bb = tile_bbox(mx, my, ex, ey, tile_bw, tile_bh, tile_h);
        uint32_t base = ci == 0 ? 0u : cum[ci - 1];
        uint32_t budget = cum[ci] - base;
        uint32_t hits = 0;
        for (uint32_t ty = bb.min_y; ty < bb.max_y && hits < budget; ty++)
            for (uint32_t tx = bb.min_x; tx < bb.max_x && hits < budget; tx++)
                if (will_contribute(tx, ty, tile_h, mx, my, conic, pt)) {
                    tile_id_from_isect[base + hits] = tx + ty * tile_bw;
                    compact_gid_from_isect[base + hits] = (uint32_t)ci;
                    hits++;
                }
        for (uint32_t k = hits; k < budget; k++) {
            tile_id_from_isect[base + k] = tile_bw * tile_bh;
            compact_gid_from_isect[base + k] = (uint32_t)ci;
        }
    }
}

/* get_tile_offsets + zero fill (get_tile_offset.rs:10-62; render.rs:396-400). */
void or_tile_offsets(const uint32_t* ids, uint64_t m, uint32_t num_tiles, uint32_t* offsets) {
    memset(offsets, 0, (size_t)num_tiles * 2 * sizeof(uint32_t));
    for (uint64_t i = 0; i < m; i++) {
        uint32_t tid = ids[i];
        if (i == 0) {
            if (tid < num_tiles) offsets[2 * tid] = 0;
        } else {
            uint32_t prev = ids[i - 1];
            if (tid != prev) {
                if (prev < num_tiles) offsets[2 * prev + 1] = (uint32_t)i;
                if (tid < num_tiles) offsets[2 * tid] = (uint32_t)i;
            }
        }
        if (i == m - 1 && tid < num_tiles) offsets[2 * tid + 1] = (uint32_t)(i + 1);
    }
}

/* ------------------------------------------------------------------------ */
/* Forward blend (kernels/rasterize.rs:24-200) with the alpha cutoff         */
/* (kernels/helpers.rs:161-190).                                             */
/* ------------------------------------------------------------------------ */
static const float CUT_MID = 1.0f / 255.0f;
static const float CUT_BAND = 1.0e-3f;

static float cutoff_weight(float alpha) {
    float t = bh_clampf((alpha - (CUT_MID - 0.5f * CUT_BAND)) / CUT_BAND, 0.0f, 1.0f);
    return t * t * (3.0f - 2.0f * t);
}
static float cutoff_weight_deriv(float alpha) {
    float low = CUT_MID - 0.5f * CUT_BAND;
    float high = CUT_MID + 0.5f * CUT_BAND;
    int inside = alpha > low && alpha < high;
    float t = (alpha - low) / CUT_BAND;
    return inside ? (6.0f * t - 6.0f * t * t) / CUT_BAND : 0.0f;
}

void or_rasterize(uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t tile_bh,
                  const float* bg, const float* projected, const uint32_t* cgid_from_isect,
                  const uint32_t* gfc, const uint32_t* off_pre, uint32_t flags, void* out_img,
                  float* visible, uint32_t* off_post) {
    int bwd_info = (flags & BH_FLAG_BWD_INFO) != 0;
    int smooth = (flags & BH_FLAG_SMOOTH_CUTOFF) != 0;
    int depth = bwd_info && (flags & BH_FLAG_RENDER_DEPTH) != 0;
    uint32_t chans = depth ? 5u : 4u;
    int64_t num_tiles = (int64_t)tile_bw * tile_bh;
    const uint32_t th = (flags & BH_FLAG_TILE_16X8) ? 8u : 16u;
#pragma omp parallel for schedule(dynamic, 4) num_threads(g_threads)
    for (int64_t tile = 0; tile < num_tiles; tile++) {
        uint32_t lo = off_pre[2 * tile], hi = off_pre[2 * tile + 1];
        uint32_t ox = (uint32_t)(tile % tile_bw) * 16u, oy = (uint32_t)(tile / tile_bw) * th;
        uint32_t max_useful = lo;
        for (uint32_t p = 0; p < 16u * th; p++) {
            uint32_t px = ox + (p & 15u), py = oy + (p >> 4);
            if (px >= img_w || py >= img_h) continue;
            float pcx = (float)px + 0.5f, pcy = (float)py + 0.5f;
            float t_acc = 1.0f, r = 0.0f, g = 0.0f, b = 0.0f, d = 0.0f;
            uint32_t last = lo;
            for (uint32_t i = lo; i < hi; i++) {
                const float* s = projected + (size_t)cgid_from_isect[i] * 10;
                /* e^-sigma in base 2 (bh_math.h: bh_power_log2, bh_exp2_neg) */
                float ca, cb, cc;
                bh_conic_log2(s[2], s[3], s[4], &ca, &cb, &cc);
                float power = bh_power_log2(ca, cb, cc, s[0] - pcx, s[1] - pcy);
                float alpha = bh_minf(0.999f, s[5] * bh_exp2_neg(-power));
                float w = smooth ? cutoff_weight(alpha) : (alpha >= CUT_MID ? 1.0f : 0.0f);
                if (power >= 0.0f && w > 0.0f) {
                    float ae = alpha * w;
                    float next_t = t_acc * (1.0f - ae);
                    if (next_t <= 1.0e-4f) break;
                    if (bwd_info) visible[gfc[cgid_from_isect[i]]] = 1.0f;
                    float vis = ae * t_acc;
                    /* pix_out += color * vis (rasterize.rs) as one fma a channel:
                     * the WGSL leaves contraction to the platform's shader
                     * compiler; this restatement and the kernels fix it as fma */
                    r = fmaf(bh_maxf(s[6], 0.0f), vis, r);
                    g = fmaf(bh_maxf(s[7], 0.0f), vis, g);
                    b = fmaf(bh_maxf(s[8], 0.0f), vis, b);
                    if (depth) d = fmaf(s[9], vis, d);
                    t_acc = next_t;
                    last = i + 1;
                }
            }
            if (last > max_useful) max_useful = last;
            float fr = r + t_acc * bg[0], fg = g + t_acc * bg[1], fb = b + t_acc * bg[2];
            float fa = 1.0f - t_acc;
            size_t pix = (size_t)py * img_w + px;
            if (bwd_info) {
                float* o = (float*)out_img + pix * chans;
                o[0] = fr; o[1] = fg; o[2] = fb; o[3] = fa;
                if (depth) o[4] = d;
            } else {
                uint32_t ur = (uint32_t)bh_clampf(fr * 255.0f, 0.0f, 255.0f);
                uint32_t ug = (uint32_t)bh_clampf(fg * 255.0f, 0.0f, 255.0f);
                uint32_t ub = (uint32_t)bh_clampf(fb * 255.0f, 0.0f, 255.0f);
                uint32_t ua = (uint32_t)bh_clampf(fa * 255.0f, 0.0f, 255.0f);
                ((uint32_t*)out_img)[pix] = ur | (ug << 8) | (ub << 16) | (ua << 24);
            }
        }
        off_post[2 * tile] = lo;
        off_post[2 * tile + 1] = bwd_info ? max_useful : hi;
    }
}

/* Independent per-pixel walk over all depth-sorted projected splats, no tiles
 * (brush-render/src/tests/raster_oracle.rs:48-98). */
void or_rasterize_reference(const float* projected, uint32_t n, uint32_t w, uint32_t h,
                            const float* bg, uint32_t smooth, float* out) {
    for (uint32_t y = 0; y < h; y++)
        for (uint32_t x = 0; x < w; x++) {
            float pxc = (float)x + 0.5f, pyc = (float)y + 0.5f;
            float t = 1.0f, r = 0.0f, g = 0.0f, b = 0.0f;
            for (uint32_t i = 0; i < n; i++) {
                const float* s = projected + (size_t)i * 10;
                float ca, cb, cc;
                bh_conic_log2(s[2], s[3], s[4], &ca, &cb, &cc);
                float power = bh_power_log2(ca, cb, cc, s[0] - pxc, s[1] - pyc);
                float alpha = bh_minf(s[5] * bh_exp2_neg(-power), 0.999f);
                float wgt = smooth ? cutoff_weight(alpha) : (alpha >= CUT_MID ? 1.0f : 0.0f);
                if (power >= 0.0f && wgt > 0.0f) {
                    float ea = alpha * wgt;
                    float nt = t * (1.0f - ea);
                    if (nt <= 1.0e-4f) break;
                    float vis = ea * t;
                    r = fmaf(bh_maxf(s[6], 0.0f), vis, r);
                    g = fmaf(bh_maxf(s[7], 0.0f), vis, g);
                    b = fmaf(bh_maxf(s[8], 0.0f), vis, b);
                    t = nt;
                }
            }
            float* o = out + ((size_t)y * w + x) * 4;
            o[0] = r + bg[0] * t;
            o[1] = g + bg[1] * t;
            o[2] = b + bg[2] * t;
            o[3] = 1.0f - t;
        }
}

/* ------------------------------------------------------------------------ */
/* Rasterize backward (brush-render-bwd/src/kernels/rasterize_backwards.rs). */
/* The reference replays each tile front to back: lane = splat, and each     */
/* splat visits the tile's 256 pixels in row-major order, carrying per-pixel */
/* state (rgb remaining, T) from splat to splat.  The per-(splat, tile)      */
/* gradient is summed over pixels in that order, then added to v_combined.   */
/* Here tiles are visited in row-major order.  The per-(splat, tile) sum is  */
/* formed as the GPU forms it: over each 64-pixel strip (tile rows 4k..4k+3) */
/* in pixel order, then strip 0 + strip 1 + strip 2 + strip 3.  The GPU adds */
/* the per-tile sums with atomics, so only the cross-tile order differs.     */
/* ------------------------------------------------------------------------ */
/* check: OR_CHECK_DROP_LAST_BATCH plants a mistake for the tests of the
 * gradient tolerance (the last 64 entries of every tile's list, or the
 * partial batch that ends it, are skipped).  v_abs (may be NULL) receives,
 * per lane, the sum over the lane's per-pixel terms of a bound on each
 * term's magnitude that also bounds the magnitudes it is computed from (see
 * or_rasterize_backward_check in bh_oracle.h). */
static void rasterize_backward_impl(uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t tile_bh,
                                    const float* bg, const float* out_img, const float* projected,
                                    const uint32_t* cgid_from_isect, const uint32_t* offsets,
                                    uint32_t num_visible, const float* v_output, uint32_t flags,
                                    float* v_combined, float* v_abs, float* v_sq, uint32_t check) {
    int smooth = (flags & BH_FLAG_SMOOTH_CUTOFF) != 0;
    int refine = (flags & BH_FLAG_REFINE_WEIGHT) != 0;
    int depth = (flags & BH_FLAG_RENDER_DEPTH) != 0;
    uint32_t chans = depth ? 5u : 4u;
    memset(v_combined, 0, (size_t)(num_visible ? num_visible : 1) * 11 * sizeof(float));
    if (v_abs) memset(v_abs, 0, (size_t)(num_visible ? num_visible : 1) * 11 * sizeof(float));
    if (v_abs) memset(v_sq, 0, (size_t)(num_visible ? num_visible : 1) * 11 * sizeof(float));
    float img_wf = (float)img_w, img_hf = (float)img_h;
    int64_t num_tiles = (int64_t)tile_bw * tile_bh;
    const uint32_t th = (flags & BH_FLAG_TILE_16X8) ? 8u : 16u;
#pragma omp parallel for schedule(dynamic, 2) num_threads(g_threads)
    for (int64_t tile = 0; tile < num_tiles; tile++) {
        uint32_t lo = offsets[2 * tile], hi = offsets[2 * tile + 1];
        if (hi <= lo) continue;
        if (check & OR_CHECK_DROP_LAST_BATCH) hi = lo + (hi - lo - 1u) / 64u * 64u;
        uint32_t ox = (uint32_t)(tile % tile_bw) * 16u, oy = (uint32_t)(tile / tile_bw) * th;
        float st[256][5];
        /* per pixel: the sum of squares of the magnitudes the remaining
         * colour has been rounded at along the walk (per channel) */
        double se[256][3];
        for (uint32_t p = 0; p < 16u * th; p++) {
            uint32_t px = ox + (p & 15u), py = oy + (p >> 4);
            if (px < img_w && py < img_h) {
                const float* o = out_img + ((size_t)py * img_w + px) * chans;
                float t_final = 1.0f - o[3];
                st[p][0] = o[0] - t_final * bg[0];
                st[p][1] = o[1] - t_final * bg[1];
                st[p][2] = o[2] - t_final * bg[2];
                st[p][3] = 1.0f;
                st[p][4] = depth ? o[4] : 0.0f;
            } else {
                st[p][0] = st[p][1] = st[p][2] = st[p][3] = st[p][4] = 0.0f;
            }
            se[p][0] = se[p][1] = se[p][2] = 0.0;
        }
        for (uint32_t i = lo; i < hi; i++) {
            uint32_t cg = cgid_from_isect[i];
            const float* s = projected + (size_t)cg * 10;
            s2 c = {s[2], s[3], s[4]};
            float ca, cbc, cc;
            bh_conic_log2(c.c00, c.c01, c.c11, &ca, &cbc, &cc);
            float cr = bh_maxf(s[6], 0.0f), cgc = bh_maxf(s[7], 0.0f), cb = bh_maxf(s[8], 0.0f);
            float gs[4][11] = {{0}};
            double ga[11] = {0}, gq[11] = {0};
            for (uint32_t p = 0; p < 16u * th; p++) {
                float* gr = gs[p >> 6];
                float sx = st[p][0], sy = st[p][1], sz = st[p][2], sw = st[p][3];
                if (!(sw > 1.0e-4f)) continue;
                uint32_t px = ox + (p & 15u), py = oy + (p >> 4);
                float pcx = (float)px + 0.5f, pcy = (float)py + 0.5f;
                float dx = s[0] - pcx, dy = s[1] - pcy;
                float power = bh_power_log2(ca, cbc, cc, dx, dy);
                float gaussian = bh_exp2_neg(-power);
                float alpha = bh_minf(0.999f, s[5] * gaussian);
                float w = smooth ? cutoff_weight(alpha) : (alpha >= CUT_MID ? 1.0f : 0.0f);
                if (!(power >= 0.0f && w > 0.0f)) continue;
                float ae = alpha * w;
                float next_t = sw * (1.0f - ae);
                if (next_t <= 1.0e-4f) {
                    st[p][3] = 0.0f;
                    continue;
                }
                float vis = ae * sw;
                const float* vo = v_output + ((size_t)py * img_w + px) * chans;
                float vox = vo[0], voy = vo[1], voz = vo[2], va = vo[3];
                float final_a = out_img[((size_t)py * img_w + px) * chans + 3];
                float t_final = 1.0f - final_a;
                float vow = (va - (bg[0] * vox + bg[1] * voy + bg[2] * voz)) * t_final;
                gr[5] += s[6] >= 0.0f ? vis * vox : 0.0f;
                gr[6] += s[7] >= 0.0f ? vis * voy : 0.0f;
                gr[7] += s[8] >= 0.0f ? vis * voz : 0.0f;
                float ra = 1.0f / (1.0f - ae);
                float dot_rgb = ((sw * cr - sx) * vox + (sw * cgc - sy) * voy + (sw * cb - sz) * voz) * ra;
                float nrx = sx - vis * cr, nry = sy - vis * cgc, nrz = sz - vis * cb;
                if (depth) {
                    float vod = vo[4];
                    float sd = st[p][4];
                    gr[10] += vis * vod;
                    st[p][4] = sd - vis * s[9];
                }
                float v_ae = dot_rgb + vow * ra;
                float dw = smooth ? cutoff_weight_deriv(alpha) : 0.0f * alpha;
                float v_alpha = v_ae * (w + alpha * dw);
                float v_sigma = -alpha * v_alpha;
                float vxy_x = v_sigma * (c.c00 * dx + c.c01 * dy);
                float vxy_y = v_sigma * (c.c01 * dx + c.c11 * dy);
                if (s[5] * gaussian <= 0.999f) {
                    gr[2] += 0.5f * v_sigma * dx * dx;
                    gr[3] += v_sigma * dx * dy;
                    gr[4] += 0.5f * v_sigma * dy * dy;
                    gr[0] += vxy_x;
                    gr[1] += vxy_y;
                    gr[8] += v_alpha * gaussian;
                    if (refine) {
                        float len = sqrtf(vxy_x * img_wf * vxy_x * img_wf + vxy_y * img_hf * vxy_y * img_hf);
                        gr[9] += len / bh_maxf(final_a, 1.0e-5f);
                    }
                }
                if (v_abs) {
                    /* the scale of the rounding noise in each term: the
                     * colour gap T c - S rounded once at its operands'
                     * magnitudes, plus the rounding S has gathered along the
                     * pixel's walk as a random walk (each step rounds a
                     * product |vis c| and a difference |S'|; the root sum of
                     * their squares), times |v_out| */
                    double m_alpha =
                        fabs((double)w + (double)alpha * dw) * (double)ra *
                        ((fabs((double)sw * cr) + fabs((double)sx) + sqrt(se[p][0])) * fabs((double)vox) +
                         (fabs((double)sw * cgc) + fabs((double)sy) + sqrt(se[p][1])) * fabs((double)voy) +
                         (fabs((double)sw * cb) + fabs((double)sz) + sqrt(se[p][2])) * fabs((double)voz) +
                         fabs((double)vow));
                    double m_sigma = (double)alpha * m_alpha;
                    double ddx = fabs((double)dx), ddy = fabs((double)dy);
                    double mt[11] = {0};
                    mt[5] = s[6] >= 0.0f ? (double)vis * fabs((double)vox) : 0.0;
                    mt[6] = s[7] >= 0.0f ? (double)vis * fabs((double)voy) : 0.0;
                    mt[7] = s[8] >= 0.0f ? (double)vis * fabs((double)voz) : 0.0;
                    if (depth) mt[10] = (double)vis * fabs((double)vo[4]);
                    if (s[5] * gaussian <= 0.999f) {
                        mt[0] = m_sigma * (fabs((double)c.c00) * ddx + fabs((double)c.c01) * ddy);
                        mt[1] = m_sigma * (fabs((double)c.c01) * ddx + fabs((double)c.c11) * ddy);
                        mt[2] = 0.5 * m_sigma * ddx * ddx;
                        mt[3] = m_sigma * ddx * ddy;
                        mt[4] = 0.5 * m_sigma * ddy * ddy;
                        mt[8] = m_alpha * (double)gaussian;
                        if (refine)
                            mt[9] = sqrt(mt[0] * img_wf * mt[0] * img_wf + mt[1] * img_hf * mt[1] * img_hf) /
                                    (double)bh_maxf(final_a, 1.0e-5f);
                    }
                    /* the terms' own magnitudes, for the summation order (the
                     * 2D-mean lanes as sums of v_sigma dx and v_sigma dy
                     * times the conic, the GPU's grouping) */
                    double at[11] = {0};
                    at[5] = mt[5], at[6] = mt[6], at[7] = mt[7], at[10] = mt[10];
                    if (s[5] * gaussian <= 0.999f) {
                        double vs = fabs((double)v_sigma);
                        at[0] = vs * (fabs((double)c.c00) * ddx + fabs((double)c.c01) * ddy);
                        at[1] = vs * (fabs((double)c.c01) * ddx + fabs((double)c.c11) * ddy);
                        at[2] = 0.5 * vs * ddx * ddx;
                        at[3] = vs * ddx * ddy;
                        at[4] = 0.5 * vs * ddy * ddy;
                        at[8] = fabs((double)v_alpha * (double)gaussian);
                        if (refine)
                            at[9] = sqrt(at[0] * img_wf * at[0] * img_wf + at[1] * img_hf * at[1] * img_hf) /
                                    (double)bh_maxf(final_a, 1.0e-5f);
                    }
                    for (int k = 0; k < 11; k++) ga[k] += at[k], gq[k] += mt[k] * mt[k];
                    double pr = (double)vis * cr, pg = (double)vis * cgc, pb = (double)vis * cb;
                    se[p][0] += pr * pr + (double)nrx * nrx;
                    se[p][1] += pg * pg + (double)nry * nry;
                    se[p][2] += pb * pb + (double)nrz * nrz;
                }
                st[p][0] = nrx;
                st[p][1] = nry;
                st[p][2] = nrz;
                st[p][3] = next_t;
            }
            float gr[11];
            for (int k = 0; k < 11; k++) gr[k] = ((gs[0][k] + gs[1][k]) + gs[2][k]) + gs[3][k];
            float* out = v_combined + (size_t)cg * 11;
            float* oa = v_abs ? v_abs + (size_t)cg * 11 : NULL;
            float* oq = v_sq ? v_sq + (size_t)cg * 11 : NULL;
            for (int k = 0; k < 11; k++) {
                if (k == 9 && !refine) continue;
                if (k == 10 && !depth) continue;
                if (g_threads > 1) {
#pragma omp atomic
                    out[k] += gr[k];
                    if (oa) {
#pragma omp atomic
                        oa[k] += (float)ga[k];
#pragma omp atomic
                        oq[k] += (float)gq[k];
                    }
                } else {
                    out[k] += gr[k];
                    if (oa) oa[k] += (float)ga[k], oq[k] += (float)gq[k];
                }
            }
        }
    }
}

void or_rasterize_backward(uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t tile_bh,
                           const float* bg, const float* out_img, const float* projected,
                           const uint32_t* cgid_from_isect, const uint32_t* offsets,
                           uint32_t num_visible, const float* v_output, uint32_t flags,
                           float* v_combined) {
    rasterize_backward_impl(img_w, img_h, tile_bw, tile_bh, bg, out_img, projected, cgid_from_isect, offsets,
                            num_visible, v_output, flags, v_combined, NULL, NULL, 0u);
}

void or_rasterize_backward_check(uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t tile_bh,
                                 const float* bg, const float* out_img, const float* projected,
                                 const uint32_t* cgid_from_isect, const uint32_t* offsets,
                                 uint32_t num_visible, const float* v_output, uint32_t flags, uint32_t check,
                                 float* v_combined, float* v_abs, float* v_sq) {
    rasterize_backward_impl(img_w, img_h, tile_bw, tile_bh, bg, out_img, projected, cgid_from_isect, offsets,
                            num_visible, v_output, flags, v_combined, v_abs, v_abs ? v_sq : NULL, check);
}

/* The same backward with every gradient quantity in double: transmittance,
 * remaining colour, the per-pixel terms and every sum.  The decisions (which
 * pairs contribute, where a pixel's walk ends) are the f32 ones above, and
 * alpha is the forward's f32 alpha, so both evaluate the gradient of the
 * same rendered image; they differ only by the f32 rounding of the
 * gradient arithmetic and of its sums.  Test infrastructure: it calibrates
 * the tolerance that the GPU backward is held to. */
void or_rasterize_backward_f64(uint32_t img_w, uint32_t img_h, uint32_t tile_bw, uint32_t tile_bh,
                               const float* bg, const float* out_img, const float* projected,
                               const uint32_t* cgid_from_isect, const uint32_t* offsets,
                               uint32_t num_visible, const float* v_output, uint32_t flags,
                               float* v_combined) {
    int smooth = (flags & BH_FLAG_SMOOTH_CUTOFF) != 0;
    int refine = (flags & BH_FLAG_REFINE_WEIGHT) != 0;
    int depth = (flags & BH_FLAG_RENDER_DEPTH) != 0;
    uint32_t chans = depth ? 5u : 4u;
    size_t rows = (size_t)(num_visible ? num_visible : 1);
    double* acc = (double*)calloc(rows * 11, sizeof(double));
    double img_wd = (double)img_w, img_hd = (double)img_h;
    int64_t num_tiles = (int64_t)tile_bw * tile_bh;
    const uint32_t th = (flags & BH_FLAG_TILE_16X8) ? 8u : 16u;
#pragma omp parallel for schedule(dynamic, 2) num_threads(g_threads)
    for (int64_t tile = 0; tile < num_tiles; tile++) {
        uint32_t lo = offsets[2 * tile], hi = offsets[2 * tile + 1];
        if (hi <= lo) continue;
        uint32_t ox = (uint32_t)(tile % tile_bw) * 16u, oy = (uint32_t)(tile / tile_bw) * th;
        float tf[256];      /* f32 transmittance: the decisions */
        double sd[256][5];  /* remaining colour, transmittance, remaining depth */
        for (uint32_t p = 0; p < 16u * th; p++) {
            uint32_t px = ox + (p & 15u), py = oy + (p >> 4);
            if (px < img_w && py < img_h) {
                const float* o = out_img + ((size_t)py * img_w + px) * chans;
                double t_final = 1.0 - (double)o[3];
                for (int k = 0; k < 3; k++) sd[p][k] = (double)o[k] - t_final * (double)bg[k];
                sd[p][3] = 1.0;
                sd[p][4] = depth ? (double)o[4] : 0.0;
                tf[p] = 1.0f;
            } else {
                for (int k = 0; k < 5; k++) sd[p][k] = 0.0;
                tf[p] = 0.0f;
            }
        }
        for (uint32_t i = lo; i < hi; i++) {
            uint32_t cg = cgid_from_isect[i];
            const float* s = projected + (size_t)cg * 10;
            float ca, cbc, cc;
            bh_conic_log2(s[2], s[3], s[4], &ca, &cbc, &cc);
            double col[3] = {(double)bh_maxf(s[6], 0.0f), (double)bh_maxf(s[7], 0.0f), (double)bh_maxf(s[8], 0.0f)};
            double g[11] = {0};
            for (uint32_t p = 0; p < 16u * th; p++) {
                float sw = tf[p];
                if (!(sw > 1.0e-4f)) continue;
                uint32_t px = ox + (p & 15u), py = oy + (p >> 4);
                float pcx = (float)px + 0.5f, pcy = (float)py + 0.5f;
                float dxf = s[0] - pcx, dyf = s[1] - pcy;
                float power = bh_power_log2(ca, cbc, cc, dxf, dyf);
                float gaussian = bh_exp2_neg(-power);
                float alpha = bh_minf(0.999f, s[5] * gaussian);
                float w = smooth ? cutoff_weight(alpha) : (alpha >= CUT_MID ? 1.0f : 0.0f);
                if (!(power >= 0.0f && w > 0.0f)) continue;
                float aef = alpha * w;
                float next_tf = sw * (1.0f - aef);
                if (next_tf <= 1.0e-4f) {
                    tf[p] = 0.0f;
                    continue;
                }
                tf[p] = next_tf;
                double T = sd[p][3], ae = (double)alpha * (double)w;
                double vis = ae * T;
                const float* vo = v_output + ((size_t)py * img_w + px) * chans;
                double vod[4] = {(double)vo[0], (double)vo[1], (double)vo[2], (double)vo[3]};
                double final_a = (double)out_img[((size_t)py * img_w + px) * chans + 3];
                double t_final = 1.0 - final_a;
                double vow = (vod[3] - ((double)bg[0] * vod[0] + (double)bg[1] * vod[1] + (double)bg[2] * vod[2])) *
                             t_final;
                for (int k = 0; k < 3; k++)
                    if (s[6 + k] >= 0.0f) g[5 + k] += vis * vod[k];
                double ra = 1.0 / (1.0 - ae);
                double dot_rgb = 0.0;
                for (int k = 0; k < 3; k++) dot_rgb += (T * col[k] - sd[p][k]) * vod[k];
                dot_rgb *= ra;
                if (depth) {
                    g[10] += vis * (double)vo[4];
                    sd[p][4] -= vis * (double)s[9];
                }
                double dw = smooth ? (double)cutoff_weight_deriv(alpha) : 0.0;
                double v_alpha = (dot_rgb + vow * ra) * ((double)w + (double)alpha * dw);
                double v_sigma = -(double)alpha * v_alpha;
                double dx = (double)dxf, dy = (double)dyf;
                double vx = v_sigma * ((double)s[2] * dx + (double)s[3] * dy);
                double vy = v_sigma * ((double)s[3] * dx + (double)s[4] * dy);
                if (s[5] * gaussian <= 0.999f) {
                    g[2] += 0.5 * v_sigma * dx * dx;
                    g[3] += v_sigma * dx * dy;
                    g[4] += 0.5 * v_sigma * dy * dy;
                    g[0] += vx;
                    g[1] += vy;
                    g[8] += v_alpha * (double)gaussian;
                    if (refine) g[9] += sqrt(vx * img_wd * vx * img_wd + vy * img_hd * vy * img_hd) /
                                        (double)bh_maxf((float)final_a, 1.0e-5f);
                }
                for (int k = 0; k < 3; k++) sd[p][k] -= vis * col[k];
                sd[p][3] = T * (1.0 - ae);
            }
            double* out = acc + (size_t)cg * 11;
            for (int k = 0; k < 11; k++) {
                if (k == 9 && !refine) continue;
                if (k == 10 && !depth) continue;
#pragma omp atomic
                out[k] += g[k];
            }
        }
    }
    for (size_t i = 0; i < rows * 11; i++) v_combined[i] = (float)acc[i];
    free(acc);
}

/* ------------------------------------------------------------------------ */
/* project_backwards (brush-render-bwd/src/kernels/project_backwards.rs)     */
/* ------------------------------------------------------------------------ */

/* Gradient through q -> q / |q| (apply_normalize_vjp, :19-52): the Jacobian
 * (I - q q^T / |q|^2) / |q| applied to g, (|q|^2 g - (q . g) q) / |q|^3.
 * Written as the product's kernels write it, so both give the same bits. */
static qt normalize_vjp(qt q, qt g) {
    float n2 = qdot(q, q);
    float qg = qdot(q, g);
    float s = 1.0f / (sqrtf(n2) * n2);
    qt r = {(n2 * g.w - qg * q.w) * s, (n2 * g.x - qg * q.x) * s, (n2 * g.y - qg * q.y) * s,
            (n2 * g.z - qg * q.z) * s};
    return r;
}
/* Gradient of sum_ab V_ab R_ab(q) through the rotation matrix of a unit
 * quaternion (quat_to_mat_vjp, :54-79): w meets the antisymmetric part of V,
 * x, y, z the symmetric part plus their own diagonal pairs. */
static qt quat_to_mat_vjp(qt q, m3 v) {
    float a_zy = v.c1z - v.c2y, a_xz = v.c2x - v.c0z, a_yx = v.c0y - v.c1x;
    float s_xy = v.c1x + v.c0y, s_xz = v.c2x + v.c0z, s_yz = v.c2y + v.c1z;
    float gw = q.x * a_zy + q.y * a_xz + q.z * a_yx;
    float gx = q.w * a_zy + q.y * s_xy + q.z * s_xz - 2.0f * q.x * (v.c1y + v.c2z);
    float gy = q.w * a_xz + q.x * s_xy + q.z * s_yz - 2.0f * q.y * (v.c0x + v.c2z);
    float gz = q.w * a_yx + q.x * s_xz + q.y * s_yz - 2.0f * q.z * (v.c0x + v.c1y);
    qt r = {2.0f * gw, 2.0f * gx, 2.0f * gy, 2.0f * gz};
    return r;
}
/* Gradient through the inverse of a symmetric 2x2 matrix (inverse2x2_vjp,
 * :81-99): dL/dM = -C V C with C = M^-1 = [[a, b], [b, c]] and V = [[p, q],
 * [q, r]], expanded entry by entry. */
static s2 inverse2x2_vjp(s2 m, s2 v) {
    float a = m.c00, b = m.c01, c = m.c11, p = v.c00, q = v.c01, r = v.c11;
    float ab = a * b, bc = b * c;
    s2 o = {-(a * a * p + 2.0f * ab * q + b * b * r), -(ab * p + (b * b + a * c) * q + bc * r),
            -(b * b * p + 2.0f * bc * q + c * c * r)};
    return o;
}
/* calculate_projection_vjp_pinhole (camera_model/pinhole.rs:58-123) */
static v3 pinhole_projection_vjp(const bh_project_uniforms* u, m23 J, v3 mean_c, s3 cov_c, s2 v_cov2d,
                         v2 v_mean2d) {
    float fx = u->fx, fy = u->fy;
    float mx = mean_c.x, my = mean_c.y, mz = mean_c.z;
    float inv_z = 1.0f / mz;
    float mx_rz_raw = mx * inv_z, my_rz_raw = my * inv_z;
    float mx_rz = bh_clampf(mx_rz_raw, u->lim_neg_x, u->lim_pos_x);
    float my_rz = bh_clampf(my_rz_raw, u->lim_neg_y, u->lim_pos_y);
    int in_x = mx_rz_raw <= u->lim_pos_x && mx_rz_raw >= u->lim_neg_x;
    int in_y = my_rz_raw <= u->lim_pos_y && my_rz_raw >= u->lim_neg_y;
    float inv_z2 = inv_z * inv_z;
    float inv_z3 = inv_z2 * inv_z;
    float v_mx = fx * inv_z * v_mean2d.x;
    float v_my = fy * inv_z * v_mean2d.y;
    float v_mz = -(fx * mx * v_mean2d.x + fy * my * v_mean2d.y) * inv_z2;
    m23 tmp = s2mulm23(v_cov2d, J);
    float vj00 = 2.0f * dot3(m23row0(tmp), s3row0(cov_c));
    float vj11 = 2.0f * dot3(m23row1(tmp), s3row1(cov_c));
    float vj20 = 2.0f * dot3(m23row0(tmp), s3row2(cov_c));
    float vj21 = 2.0f * dot3(m23row1(tmp), s3row2(cov_c));
    float tx = mz * mx_rz;
    float ty = mz * my_rz;
    if (in_x) v_mx += -fx * inv_z2 * vj20;
    else v_mz += -fx * inv_z3 * vj20 * tx;
    if (in_y) v_my += -fy * inv_z2 * vj21;
    else v_mz += -fy * inv_z3 * vj21 * ty;
    v_mz += -fx * inv_z2 * vj00 - fy * inv_z2 * vj11 + 2.0f * fx * tx * inv_z3 * vj20 + 2.0f * fy * ty * inv_z3 * vj21;
    return mk3(v_mx, v_my, v_mz);
}
/* 2 (v_cov2d J) cov_c as rows u (o[0..2]) and v (o[3..5]) */
static void cov_jac_grad(m23 J, s3 cov_c, s2 v_cov2d, float* o) {
    m23 tmp = s2mulm23(v_cov2d, J);
    o[0] = 2.0f * dot3(m23row0(tmp), s3row0(cov_c));
    o[1] = 2.0f * dot3(m23row0(tmp), s3row1(cov_c));
    o[2] = 2.0f * dot3(m23row0(tmp), s3row2(cov_c));
    o[3] = 2.0f * dot3(m23row1(tmp), s3row0(cov_c));
    o[4] = 2.0f * dot3(m23row1(tmp), s3row1(cov_c));
    o[5] = 2.0f * dot3(m23row1(tmp), s3row2(cov_c));
}
/* calculate_projection_vjp_kb4 (kannala_brandt_4.rs:138-337) */
static v3 kb4_projection_vjp(const bh_project_uniforms* u, m23 J, v3 mean_c, s3 cov_c, s2 v_cov2d, v2 v_mean2d) {
    const float* k = u->camera_params;
    float fx = u->fx, fy = u->fy, mx = mean_c.x, my = mean_c.y, mz = mean_c.z;
    float r2 = mx * mx + my * my;
    float r = bh_maxf(sqrtf(r2), 1.0e-8f);
    float rho2 = r2 + mz * mz;
    float th = bh_atan2f(r, mz);
    float th2 = th * th, th4 = th2 * th2, th6 = th4 * th2, th8 = th4 * th4;
    float theta_d = th * (1.0f + k[0] * th2 + k[1] * th4 + k[2] * th6 + k[3] * th8);
    float p1 = 1.0f + 3.0f * k[0] * th2 + 5.0f * k[1] * th4 + 7.0f * k[2] * th6 + 9.0f * k[3] * th8;
    float p2 = 6.0f * k[0] * th + 20.0f * k[1] * th * th2 + 42.0f * k[2] * th * th4 + 72.0f * k[3] * th * th6;
    float inv_r = 1.0f / r;
    float inv_r3 = inv_r * inv_r * inv_r;
    float inv_r5 = inv_r3 * inv_r * inv_r;
    float inv_rho2 = 1.0f / rho2;
    float inv_rho2_sq = inv_rho2 * inv_rho2;
    float inv_rho2_r = inv_rho2 * inv_r;
    float dth_x = mx * mz * inv_rho2_r, dth_y = my * mz * inv_rho2_r, dth_z = -r * inv_rho2;
    float xr = mx * inv_r, yr = my * inv_r;
    float dxr_x = my * my * inv_r3, dxr_y = -mx * my * inv_r3;
    float dyr_x = dxr_y, dyr_y = mx * mx * inv_r3;
    float dg_x = p1 * dth_x, dg_y = p1 * dth_y, dg_z = p1 * dth_z;
    float v_mx = dot2(v_mean2d, J.c0), v_my = dot2(v_mean2d, J.c1), v_mz = dot2(v_mean2d, J.c2);
    float vj[6];
    cov_jac_grad(J, cov_c, v_cov2d, vj);
    float three_r2_z2 = 3.0f * r2 + mz * mz;
    float r2_minus_z2 = r2 - mz * mz;
    float h00 = mz * (r2 * rho2 - mx * mx * three_r2_z2) * inv_r3 * inv_rho2_sq;
    float h11 = mz * (r2 * rho2 - my * my * three_r2_z2) * inv_r3 * inv_rho2_sq;
    float h01 = -mx * my * mz * three_r2_z2 * inv_r3 * inv_rho2_sq;
    float h02 = mx * r2_minus_z2 * inv_r * inv_rho2_sq;
    float h12 = my * r2_minus_z2 * inv_r * inv_rho2_sq;
    float h22 = 2.0f * mz * r * inv_rho2_sq;
    float two_x2_my2 = 2.0f * mx * mx - my * my;
    float two_y2_mx2 = 2.0f * my * my - mx * mx;
    float hx00 = -3.0f * mx * my * my * inv_r5;
    float hx01 = my * two_x2_my2 * inv_r5;
    float hx11 = mx * two_y2_mx2 * inv_r5;
    float hy00 = my * two_x2_my2 * inv_r5;
    float hy01 = mx * two_y2_mx2 * inv_r5;
    float hy11 = -3.0f * mx * mx * my * inv_r5;
    float d2g, du, dv;
    /* d/dx: j = 0, 1, 2 */
    d2g = p2 * dth_x * dth_x + p1 * h00;
    du = fx * (d2g * xr + dg_x * dxr_x + dg_x * dxr_x + theta_d * hx00);
    dv = fy * (d2g * yr + dg_x * dyr_x + dg_x * dyr_x + theta_d * hy00);
    v_mx += vj[0] * du + vj[3] * dv;
    d2g = p2 * dth_y * dth_x + p1 * h01;
    du = fx * (d2g * xr + dg_y * dxr_x + dg_x * dxr_y + theta_d * hx01);
    dv = fy * (d2g * yr + dg_y * dyr_x + dg_x * dyr_y + theta_d * hy01);
    v_mx += vj[1] * du + vj[4] * dv;
    d2g = p2 * dth_z * dth_x + p1 * h02;
    du = fx * (d2g * xr + dg_x * 0.0f + dg_z * dxr_x);
    dv = fy * (d2g * yr + dg_x * 0.0f + dg_z * dyr_x);
    v_mx += vj[2] * du + vj[5] * dv;
    /* d/dy */
    d2g = p2 * dth_x * dth_y + p1 * h01;
    du = fx * (d2g * xr + dg_x * dxr_y + dg_y * dxr_x + theta_d * hx01);
    dv = fy * (d2g * yr + dg_x * dyr_y + dg_y * dyr_x + theta_d * hy01);
    v_my += vj[0] * du + vj[3] * dv;
    d2g = p2 * dth_y * dth_y + p1 * h11;
    du = fx * (d2g * xr + dg_y * dxr_y + dg_y * dxr_y + theta_d * hx11);
    dv = fy * (d2g * yr + dg_y * dyr_y + dg_y * dyr_y + theta_d * hy11);
    v_my += vj[1] * du + vj[4] * dv;
    d2g = p2 * dth_z * dth_y + p1 * h12;
    du = fx * (d2g * xr + dg_y * 0.0f + dg_z * dxr_y);
    dv = fy * (d2g * yr + dg_y * 0.0f + dg_z * dyr_y);
    v_my += vj[2] * du + vj[5] * dv;
    /* d/dz */
    d2g = p2 * dth_x * dth_z + p1 * h02;
    du = fx * (d2g * xr + dg_z * dxr_x + dg_x * 0.0f);
    dv = fy * (d2g * yr + dg_z * dyr_x + dg_x * 0.0f);
    v_mz += vj[0] * du + vj[3] * dv;
    d2g = p2 * dth_y * dth_z + p1 * h12;
    du = fx * (d2g * xr + dg_z * dxr_y + dg_y * 0.0f);
    dv = fy * (d2g * yr + dg_z * dyr_y + dg_y * 0.0f);
    v_mz += vj[1] * du + vj[4] * dv;
    d2g = p2 * dth_z * dth_z + p1 * h22;
    du = fx * (d2g * xr);
    dv = fy * (d2g * yr);
    v_mz += vj[2] * du + vj[5] * dv;
    return mk3(v_mx, v_my, v_mz);
}
/* calculate_projection_vjp_rt8 (radial_tangential_8.rs:148-377) */
static v3 rt8_projection_vjp(const bh_project_uniforms* u, v3 mean_c, s3 cov_c, s2 v_cov2d, v2 v_mean2d) {
    const float* k = u->camera_params;
    float p1 = k[6], p2 = k[7], fx = u->fx, fy = u->fy;
    float mx = mean_c.x, my = mean_c.y, mz = mean_c.z;
    float inv_z = 1.0f / mz;
    float rx_raw = mx * inv_z, ry_raw = my * inv_z;
    float mx_rz = bh_clampf(rx_raw, u->lim_neg_x, u->lim_pos_x);
    float my_rz = bh_clampf(ry_raw, u->lim_neg_y, u->lim_pos_y);
    int in_x = rx_raw <= u->lim_pos_x && rx_raw >= u->lim_neg_x;
    int in_y = ry_raw <= u->lim_pos_y && ry_raw >= u->lim_neg_y;
    float xc = mx_rz * mz, yc = my_rz * mz;
    float inv_z2 = inv_z * inv_z;
    float inv_z3 = inv_z2 * inv_z;
    float x = xc * inv_z, y = yc * inv_z;
    float r2 = x * x + y * y;
    float r4 = r2 * r2;
    float n = 1.0f + k[0] * r2 + k[1] * r4 + k[2] * r2 * r4;
    float dn = 1.0f + k[3] * r2 + k[4] * r4 + k[5] * r2 * r4;
    float np = k[0] + 2.0f * k[1] * r2 + 3.0f * k[2] * r4;
    float dnp = k[3] + 2.0f * k[4] * r2 + 3.0f * k[5] * r4;
    float npp = 2.0f * k[1] + 6.0f * k[2] * r2;
    float dnpp = 2.0f * k[4] + 6.0f * k[5] * r2;
    float inv_dn = 1.0f / dn;
    float inv_dn2 = inv_dn * inv_dn;
    float inv_dn3 = inv_dn2 * inv_dn;
    float rr = n * inv_dn;
    float rrp = (np * dn - n * dnp) * inv_dn2;
    float rrpp = (npp * dn * dn - 2.0f * np * dn * dnp - n * dnpp * dn + 2.0f * n * dnp * dnp) * inv_dn3;
    float rx = 2.0f * x * rrp, ry = 2.0f * y * rrp;
    float rpx = 2.0f * x * rrpp, rpy = 2.0f * y * rrpp;
    float d00 = rr + 2.0f * x * x * rrp + 2.0f * p1 * y + 6.0f * p2 * x;
    float d01 = 2.0f * x * y * rrp + 2.0f * p1 * x + 2.0f * p2 * y;
    float d10 = d01;
    float d11 = rr + 2.0f * y * y * rrp + 6.0f * p1 * y + 2.0f * p2 * x;
    float js00 = fx * d00 * inv_z, js01 = fx * d01 * inv_z, js02 = -fx * (d00 * xc + d01 * yc) * inv_z2;
    float js10 = fy * d10 * inv_z, js11 = fy * d11 * inv_z, js12 = -fy * (d10 * xc + d11 * yc) * inv_z2;
    float je00 = in_x ? js00 : 0.0f, je10 = in_x ? js10 : 0.0f;
    float je01 = in_y ? js01 : 0.0f, je11 = in_y ? js11 : 0.0f;
    float je02 = (in_x ? 0.0f : mx_rz * js00) + (in_y ? 0.0f : my_rz * js01) + js02;
    float je12 = (in_x ? 0.0f : mx_rz * js10) + (in_y ? 0.0f : my_rz * js11) + js12;
    float v_mx = je00 * v_mean2d.x + je10 * v_mean2d.y;
    float v_my = je01 * v_mean2d.x + je11 * v_mean2d.y;
    float v_mz = je02 * v_mean2d.x + je12 * v_mean2d.y;
    float ve[6];
    cov_jac_grad(mkm23(je00, je10, je01, je11, je02, je12), cov_c, v_cov2d, ve);
    float su0 = in_x ? ve[0] : mx_rz * ve[2], sv0 = in_x ? ve[3] : mx_rz * ve[5];
    float su1 = in_y ? ve[1] : my_rz * ve[2], sv1 = in_y ? ve[4] : my_rz * ve[5];
    float su2 = ve[2], sv2 = ve[5];
    float a00x = rx + 4.0f * x * rrp + 2.0f * x * x * rpx + 6.0f * p2;
    float a00y = ry + 2.0f * x * x * rpy + 2.0f * p1;
    float a01x = 2.0f * y * rrp + 2.0f * x * y * rpx + 2.0f * p1;
    float a01y = 2.0f * x * rrp + 2.0f * x * y * rpy + 2.0f * p2;
    float a10x = a01x, a10y = a01y;
    float a11x = rx + 2.0f * y * y * rpx + 2.0f * p2;
    float a11y = ry + 4.0f * y * rrp + 2.0f * y * y * rpy + 6.0f * p1;
    float b00xc = a00x * inv_z, b00yc = a00y * inv_z, b00z = -(xc * a00x + yc * a00y) * inv_z2;
    float b01xc = a01x * inv_z, b01yc = a01y * inv_z, b01z = -(xc * a01x + yc * a01y) * inv_z2;
    float b10xc = a10x * inv_z, b10yc = a10y * inv_z, b10z = -(xc * a10x + yc * a10y) * inv_z2;
    float b11xc = a11x * inv_z, b11yc = a11y * inv_z, b11z = -(xc * a11x + yc * a11y) * inv_z2;
    float j00xc = fx * b00xc * inv_z, j00yc = fx * b00yc * inv_z, j00z = fx * (b00z * inv_z - d00 * inv_z2);
    float j01xc = fx * b01xc * inv_z, j01yc = fx * b01yc * inv_z, j01z = fx * (b01z * inv_z - d01 * inv_z2);
    float j10xc = fy * b10xc * inv_z, j10yc = fy * b10yc * inv_z, j10z = fy * (b10z * inv_z - d10 * inv_z2);
    float j11xc = fy * b11xc * inv_z, j11yc = fy * b11yc * inv_z, j11z = fy * (b11z * inv_z - d11 * inv_z2);
    float j02xc = -fx * (b00xc * xc + d00 + b01xc * yc) * inv_z2;
    float j02yc = -fx * (b00yc * xc + b01yc * yc + d01) * inv_z2;
    float j02z = -fx * ((b00z * xc + b01z * yc) * inv_z2 - 2.0f * (d00 * xc + d01 * yc) * inv_z3);
    float j12xc = -fy * (b10xc * xc + d10 + b11xc * yc) * inv_z2;
    float j12yc = -fy * (b10yc * xc + b11yc * yc + d11) * inv_z2;
    float j12z = -fy * ((b10z * xc + b11z * yc) * inv_z2 - 2.0f * (d10 * xc + d11 * yc) * inv_z3);
    float c_xc = su0 * j00xc + su1 * j01xc + su2 * j02xc + sv0 * j10xc + sv1 * j11xc + sv2 * j12xc;
    float c_yc = su0 * j00yc + su1 * j01yc + su2 * j02yc + sv0 * j10yc + sv1 * j11yc + sv2 * j12yc;
    float c_z = su0 * j00z + su1 * j01z + su2 * j02z + sv0 * j10z + sv1 * j11z + sv2 * j12z;
    if (in_x) v_mx += c_xc;
    if (in_y) v_my += c_yc;
    v_mz += c_z;
    if (!in_x) v_mz += mx_rz * c_xc;
    if (!in_y) v_mz += my_rz * c_yc;
    return mk3(v_mx, v_my, v_mz);
}
/* calculate_projection_vjp_tpf (thin_prism_fisheye.rs:116-203) */
static v3 tpf_projection_vjp(const bh_project_uniforms* u, m23 J, v3 mean_c, s3 cov_c, s2 v_cov2d, v2 v_mean2d) {
    v3 kb = kb4_projection_vjp(u, J, mean_c, cov_c, v_cov2d, v_mean2d);
    float p1 = u->camera_params[4], p2 = u->camera_params[5];
    float sx1 = u->camera_params[6], sy1 = u->camera_params[7];
    float fx = u->fx, fy = u->fy;
    float inv_z = 1.0f / mean_c.z;
    float inv_z2 = inv_z * inv_z;
    float inv_z3 = inv_z2 * inv_z;
    float inv_z4 = inv_z2 * inv_z2;
    float t[6];
    tpf_polys(u, mean_c.x, mean_c.y, t);
    float hu00 = (6.0f * p2 + 2.0f * sx1) * inv_z2, hu01 = (2.0f * p1) * inv_z2, hu11 = (2.0f * p2 + 2.0f * sx1) * inv_z2;
    float hu02 = -2.0f * t[2] * inv_z3, hu12 = -2.0f * t[3] * inv_z3, hu22 = 6.0f * t[0] * inv_z4;
    float hv00 = (2.0f * p1 + 2.0f * sy1) * inv_z2, hv01 = (2.0f * p2) * inv_z2, hv11 = (6.0f * p1 + 2.0f * sy1) * inv_z2;
    float hv02 = -2.0f * t[4] * inv_z3, hv12 = -2.0f * t[5] * inv_z3, hv22 = 6.0f * t[1] * inv_z4;
    float vj[6];
    cov_jac_grad(J, cov_c, v_cov2d, vj);
    float ax = fx * (vj[0] * hu00 + vj[1] * hu01 + vj[2] * hu02) + fy * (vj[3] * hv00 + vj[4] * hv01 + vj[5] * hv02);
    float ay = fx * (vj[0] * hu01 + vj[1] * hu11 + vj[2] * hu12) + fy * (vj[3] * hv01 + vj[4] * hv11 + vj[5] * hv12);
    float az = fx * (vj[0] * hu02 + vj[1] * hu12 + vj[2] * hu22) + fy * (vj[3] * hv02 + vj[4] * hv12 + vj[5] * hv22);
    return mk3(kb.x + ax, kb.y + ay, kb.z + az);
}
/* calculate_projection_vjp (camera_model/mod.rs:82-126) */
static v3 cam_projection_vjp(const bh_project_uniforms* u, m23 J, v3 mean_c, s3 cov_c, s2 v_cov2d, v2 v_mean2d) {
    switch (u->camera_model) {
        case BH_CAMERA_KB4: return kb4_projection_vjp(u, J, mean_c, cov_c, v_cov2d, v_mean2d);
        case BH_CAMERA_RT8: return rt8_projection_vjp(u, mean_c, cov_c, v_cov2d, v_mean2d);
        case BH_CAMERA_TPF: return tpf_projection_vjp(u, J, mean_c, cov_c, v_cov2d, v_mean2d);
        default: return pinhole_projection_vjp(u, J, mean_c, cov_c, v_cov2d, v_mean2d);
    }
}

/* Test hooks: the camera models on their own. */
void or_atan2f(const float* y, const float* x, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = bh_atan2f(y[i], x[i]);
}
void or_camera_project(const bh_project_uniforms* u, const float* pts, uint64_t n, float* out, uint8_t* culled) {
    for (uint64_t i = 0; i < n; i++) {
        v3 p = mk3(pts[3 * i], pts[3 * i + 1], pts[3 * i + 2]);
        project_point(u, p, &out[2 * i], &out[2 * i + 1]);
        culled[i] = (uint8_t)depth_culled(u, p);
    }
}
void or_camera_jacobian(const bh_project_uniforms* u, const float* pts, uint64_t n, float* out) {
    for (uint64_t i = 0; i < n; i++) {
        m23 J = cam_jacobian(u, mk3(pts[3 * i], pts[3 * i + 1], pts[3 * i + 2]));
        float* o = out + 6 * i;
        o[0] = J.c0.x; o[1] = J.c1.x; o[2] = J.c2.x;
        o[3] = J.c0.y; o[4] = J.c1.y; o[5] = J.c2.y;
    }
}
/* cov_c rows c00 c01 c02 c11 c12 c22; v_cov2d c00 c01 c11 */
void or_camera_vjp(const bh_project_uniforms* u, const float* mean_c, const float* cov_c, const float* v_cov2d,
                   const float* v_mean2d, uint64_t n, float* out) {
    for (uint64_t i = 0; i < n; i++) {
        v3 m = mk3(mean_c[3 * i], mean_c[3 * i + 1], mean_c[3 * i + 2]);
        const float* c = cov_c + 6 * i;
        s3 cc = {c[0], c[1], c[2], c[3], c[4], c[5]};
        s2 vc = {v_cov2d[3 * i], v_cov2d[3 * i + 1], v_cov2d[3 * i + 2]};
        v3 g = cam_projection_vjp(u, cam_jacobian(u, m), m, cc, vc, mk2(v_mean2d[2 * i], v_mean2d[2 * i + 1]));
        out[3 * i] = g.x;
        out[3 * i + 1] = g.y;
        out[3 * i + 2] = g.z;
    }
}
/* sh_coeffs_to_color_vjp (kernels/sh.rs:383-466) */
static void wr3(float* o, uint32_t k, v3 v) {
    o[3 * k] = v.x;
    o[3 * k + 1] = v.y;
    o[3 * k + 2] = v.z;
}
static void sh_color_vjp(float* o, uint32_t deg, v3 v, v3 vc) {
    wr3(o, 0, scl3(vc, 0.2820948f));
    if (deg >= 1) {
        float f0a = 0.4886025f;
        wr3(o, 1, scl3(vc, -f0a * v.y));
        wr3(o, 2, scl3(vc, f0a * v.z));
        wr3(o, 3, scl3(vc, -f0a * v.x));
        if (deg >= 2) {
            float z2 = v.z * v.z;
            float f0b = -1.0925485f * v.z;
            float f1a = 0.54627424f;
            float fc1 = v.x * v.x - v.y * v.y;
            float fs1 = 2.0f * v.x * v.y;
            float p6 = 0.9461747f * z2 - 0.31539157f;
            wr3(o, 4, scl3(vc, f1a * fs1));
            wr3(o, 5, scl3(vc, f0b * v.y));
            wr3(o, 6, scl3(vc, p6));
            wr3(o, 7, scl3(vc, f0b * v.x));
            wr3(o, 8, scl3(vc, f1a * fc1));
            if (deg >= 3) {
                float f0c = -2.285229f * z2 + 0.4570458f;
                float f1b = 1.4453057f * v.z;
                float f2a = -0.5900436f;
                float fc2 = v.x * fc1 - v.y * fs1;
                float fs2 = v.x * fs1 + v.y * fc1;
                float p12 = v.z * (1.8658817f * z2 - 1.119529f);
                wr3(o, 9, scl3(vc, f2a * fs2));
                wr3(o, 10, scl3(vc, f1b * fs1));
                wr3(o, 11, scl3(vc, f0c * v.y));
                wr3(o, 12, scl3(vc, p12));
                wr3(o, 13, scl3(vc, f0c * v.x));
                wr3(o, 14, scl3(vc, f1b * fc1));
                wr3(o, 15, scl3(vc, f2a * fc2));
                if (deg >= 4) {
                    float f0d = v.z * (-4.683326f * z2 + 2.0071396f);
                    float f1c = 3.3116114f * z2 - 0.47308735f;
                    float f2b = -1.7701308f * v.z;
                    float f3a = 0.62583575f;
                    float fc3 = v.x * fc2 - v.y * fs2;
                    float fs3 = v.x * fs2 + v.y * fc2;
                    float p20 = 1.9843135f * v.z * p12 + -1.0062306f * p6;
                    wr3(o, 16, scl3(vc, f3a * fs3));
                    wr3(o, 17, scl3(vc, f2b * fs2));
                    wr3(o, 18, scl3(vc, f1c * fs1));
                    wr3(o, 19, scl3(vc, f0d * v.y));
                    wr3(o, 20, scl3(vc, p20));
                    wr3(o, 21, scl3(vc, f0d * v.x));
                    wr3(o, 22, scl3(vc, f1c * fc1));
                    wr3(o, 23, scl3(vc, f2b * fc2));
                    wr3(o, 24, scl3(vc, f3a * fc3));
                }
            }
        }
    }
}
/* The z factor F(z) of the degree-l, order-m SH basis functions and dF/dz:
 * every basis function of sh_to_color is F(z) times Re or Im of (x + i y)^m
 * (cosine part at index l^2 + l + m, sine part at l^2 + l - m). */
static void sh_z_factor(int l, int m, float z, float* f, float* df) {
    float z2 = z * z;
    switch (l * 8 + m) {
        case 8: *f = 0.4886025f * z, *df = 0.4886025f; break;
        case 9: *f = -0.4886025f, *df = 0.0f; break;
        case 16: *f = 0.9461747f * z2 - 0.31539157f, *df = 1.8923494f * z; break;
        case 17: *f = -1.0925485f * z, *df = -1.0925485f; break;
        case 18: *f = 0.54627424f, *df = 0.0f; break;
        case 24: *f = z * (1.8658817f * z2 - 1.119529f), *df = 5.5976451f * z2 - 1.119529f; break;
        case 25: *f = -2.285229f * z2 + 0.4570458f, *df = -4.570458f * z; break;
        case 26: *f = 1.4453057f * z, *df = 1.4453057f; break;
        case 27: *f = -0.5900436f, *df = 0.0f; break;
        case 32: {
            float f3 = z * (1.8658817f * z2 - 1.119529f), d3 = 5.5976451f * z2 - 1.119529f;
            float f2 = 0.9461747f * z2 - 0.31539157f, d2 = 1.8923494f * z;
            *f = 1.9843135f * z * f3 - 1.0062306f * f2;
            *df = 1.9843135f * (f3 + z * d3) - 1.0062306f * d2;
            break;
        }
        case 33: *f = z * (-4.683326f * z2 + 2.0071396f), *df = -14.049978f * z2 + 2.0071396f; break;
        case 34: *f = 3.3116114f * z2 - 0.47308735f, *df = 6.6232228f * z; break;
        case 35: *f = -1.7701308f * z, *df = -1.7701308f; break;
        default: *f = 0.62583575f, *df = 0.0f; break;
    }
}
/* The colour's gradient with respect to the view direction (the derivative
 * sh_color_viewdir_vjp, kernels/sh.rs:249-381, takes term by term): a pair of
 * order m with weights wc, ws (the coefficient rows dotted with the colour
 * gradient) adds F m (wc C + ws S, ws C - wc S) with C + i S = (x + i y)^(m-1)
 * to x and y, and F' (wc Re + ws Im)((x + i y)^m) to z. */
static v3 sh_viewdir_vjp(const float* c, uint32_t deg, v3 v, v3 vc) {
    float re[5], im[5];
    re[0] = 1.0f, im[0] = 0.0f;
    for (uint32_t m = 1; m <= deg; m++) {
        re[m] = v.x * re[m - 1] - v.y * im[m - 1];
        im[m] = v.x * im[m - 1] + v.y * re[m - 1];
    }
    float gx = 0.0f, gy = 0.0f, gz = 0.0f;
    for (int l = 1; l <= (int)deg; l++) {
        int k0 = l * l + l;
        float f, df;
        sh_z_factor(l, 0, v.z, &f, &df);
        gz += df * dot3(rd3(c, (uint32_t)k0), vc);
        for (int m = 1; m <= l; m++) {
            sh_z_factor(l, m, v.z, &f, &df);
            float wc = dot3(rd3(c, (uint32_t)(k0 + m)), vc), ws = dot3(rd3(c, (uint32_t)(k0 - m)), vc);
            float fm = f * (float)m;
            gx += fm * (wc * re[m - 1] + ws * im[m - 1]);
            gy += fm * (ws * re[m - 1] - wc * im[m - 1]);
            gz += df * (wc * re[m] + ws * im[m]);
        }
    }
    return mk3(gx, gy, gz);
}

void or_project_backward(const bh_project_uniforms* u, const float* transforms,
                         const float* sh_coeffs, const float* raw_opac,
                         const uint32_t* gfc, uint32_t num_visible, uint32_t num_splats,
                         uint32_t sh_degree, uint32_t mip, const float* v_combined,
                         float* v_transforms, float* v_coeffs, float* v_raw_opac,
                         float* v_refine) {
    uint32_t nc = (sh_degree + 1) * (sh_degree + 1);
    memset(v_transforms, 0, (size_t)num_splats * 10 * sizeof(float));
    memset(v_coeffs, 0, (size_t)num_splats * nc * 3 * sizeof(float));
    memset(v_raw_opac, 0, (size_t)num_splats * sizeof(float));
    memset(v_refine, 0, (size_t)num_splats * sizeof(float));
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int64_t ci = 0; ci < (int64_t)num_visible; ci++) {
        uint32_t g = gfc[ci];
        const float* rg = v_combined + (size_t)ci * 11;
        int any = 0;
        for (int k = 0; k < 11; k++) any |= rg[k] != 0.0f;
        if (!any) continue;
        const float* t = transforms + (size_t)g * 10;
        v3 mean = mk3(t[0], t[1], t[2]);
        v3 scale = mk3(bh_expf(t[7]), bh_expf(t[8]), bh_expf(t[9]));
        qt qu = {t[3], t[4], t[5], t[6]};
        qt q = qnormalize(qu);
        v3 uw = sub3(mean, mk3(u->camera_pos[0], u->camera_pos[1], u->camera_pos[2]));
        float ulen = len3(uw);
        v3 v = scl3(uw, 1.0f / ulen);
        const float* coeffs = sh_coeffs + (size_t)g * nc * 3;
        v3 vcol = mk3(rg[5], rg[6], rg[7]);
        sh_color_vjp(v_coeffs + (size_t)g * nc * 3, sh_degree, v, vcol);
        v3 vv = sh_viewdir_vjp(coeffs, sh_degree, v, vcol);
        float vdot = dot3(v, vv);
        v3 v_mean_sh = scl3(sub3(vv, scl3(v, vdot)), 1.0f / ulen);
        v3 mean_c = world_to_cam(u, mean);
        m3 r = qmat(q);
        m3 m = m3diag(r, scale);
        s2 raw_cov = calc_cov2d(u, scale, q, mean_c);
        float comp;
        s2 cov = compensate_cov2d(raw_cov, mip, &comp);
        float sig = bh_sigmoidf(raw_opac[g]);
        v_raw_opac[g] = comp * rg[8] * sig * (1.0f - sig);
        float rc = bh_is_finite(rg[9]) ? rg[9] : 0.0f;
        v_refine[g] = bh_clampf(rc, 0.0f, 1.0e32f);
        s2 conic_inv = s2inv(cov);
        s2 v_inv = {rg[2], rg[3] * 0.5f, rg[4]};
        s2 v_cov2d = inverse2x2_vjp(conic_inv, v_inv);
        s3 covar = m3outer(m);
        m3 vr = view_rot(u);
        s3 cov_c = s3cong(covar, vr);
        m23 J = cam_jacobian(u, mean_c);
        v3 v_mean_c = cam_projection_vjp(u, J, mean_c, cov_c, v_cov2d, mk2(rg[0], rg[1]));
        v_mean_c = mk3(v_mean_c.x, v_mean_c.y, v_mean_c.z + rg[10]);
        s3 vcc = m23tcong(J, v_cov2d);
        v3 v_mean = add3(m3tmulv(vr, v_mean_c), v_mean_sh);
        m3 v_m = s3mulm3(s3scale(s3tcong(vcc, vr), 2.0f), m);
        v3 v_scale = mk3(dot3(col0(r), col0(v_m)) * scale.x, dot3(col1(r), col1(v_m)) * scale.y,
                         dot3(col2(r), col2(v_m)) * scale.z);
        qt qg = quat_to_mat_vjp(q, m3diag(v_m, scale));
        qt vq = normalize_vjp(qu, qg);
        float* o = v_transforms + (size_t)g * 10;
        o[0] = v_mean.x; o[1] = v_mean.y; o[2] = v_mean.z;
        o[3] = vq.w; o[4] = vq.x; o[5] = vq.y; o[6] = vq.z;
        o[7] = v_scale.x; o[8] = v_scale.y; o[9] = v_scale.z;
    }
}
