// bh_splat_math.h — per-splat math of the rasterizer for gfx950 kernels.
//
// Restates the reference's cube-side math (crates/brush-cube/src/lib.rs,
// crates/brush-render/src/kernels/{helpers,sh,camera_model/pinhole}.rs,
// crates/brush-render-bwd/src/kernels/project_backwards.rs).  Expressions keep
// the reference's evaluation order and are compiled without contraction
// (-ffp-contract=off), so the integer decisions derived from them (culling,
// tile counts, tile ids) are reproducible bit for bit on a CPU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/brush_hip.h"
#include "bh_math.h"

#define BH_DEV __device__ __forceinline__

namespace bh {

struct V3 {
    float x, y, z;
};
struct V2 {
    float x, y;
};
struct Q4 {
    float w, x, y, z;
};
// 3x3, column-major: cI_R is column I, row R.
struct M3 {
    float c0x, c0y, c0z, c1x, c1y, c1z, c2x, c2y, c2z;
};
struct M23 {
    V2 c0, c1, c2;
};
struct S2 {
    float c00, c01, c11;
};
struct S3 {
    float c00, c01, c02, c11, c12, c22;
};

BH_DEV V3 v3(float x, float y, float z) { return V3{x, y, z}; }
BH_DEV V2 v2(float x, float y) { return V2{x, y}; }
BH_DEV V3 operator+(V3 a, V3 b) { return v3(a.x + b.x, a.y + b.y, a.z + b.z); }
BH_DEV V3 operator-(V3 a, V3 b) { return v3(a.x - b.x, a.y - b.y, a.z - b.z); }
BH_DEV V3 operator*(V3 a, float s) { return v3(a.x * s, a.y * s, a.z * s); }
BH_DEV float dot(V3 a, V3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
BH_DEV bool finite3(V3 a) { return bh_is_finite(a.x) && bh_is_finite(a.y) && bh_is_finite(a.z); }
BH_DEV V2 operator+(V2 a, V2 b) { return v2(a.x + b.x, a.y + b.y); }
BH_DEV V2 operator*(V2 a, float s) { return v2(a.x * s, a.y * s); }
BH_DEV float dot(V2 a, V2 b) { return a.x * b.x + a.y * b.y; }

BH_DEV float qdot(Q4 a, Q4 b) { return a.w * b.w + a.x * b.x + a.y * b.y + a.z * b.z; }
// Quat::normalize (lib.rs:185-188)
BH_DEV Q4 qnormalize(Q4 q) {
    float s = 1.0f / sqrtf(qdot(q, q));
    return Q4{q.w * s, q.x * s, q.y * s, q.z * s};
}
// Quat::to_mat3 (lib.rs:190-216)
BH_DEV M3 qmat(Q4 q) {
    float x2 = q.x * q.x, y2 = q.y * q.y, z2 = q.z * q.z;
    float xy = q.x * q.y, xz = q.x * q.z, yz = q.y * q.z;
    float wx = q.w * q.x, wy = q.w * q.y, wz = q.w * q.z;
    M3 m;
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
BH_DEV V3 col0(const M3& m) { return v3(m.c0x, m.c0y, m.c0z); }
BH_DEV V3 col1(const M3& m) { return v3(m.c1x, m.c1y, m.c1z); }
BH_DEV V3 col2(const M3& m) { return v3(m.c2x, m.c2y, m.c2z); }
BH_DEV V3 row0(const M3& m) { return v3(m.c0x, m.c1x, m.c2x); }
BH_DEV V3 row1(const M3& m) { return v3(m.c0y, m.c1y, m.c2y); }
BH_DEV V3 row2(const M3& m) { return v3(m.c0z, m.c1z, m.c2z); }
BH_DEV M3 from_cols(V3 a, V3 b, V3 c) { return M3{a.x, a.y, a.z, b.x, b.y, b.z, c.x, c.y, c.z}; }
// Mat3::mul_vec3 (lib.rs:262-268)
BH_DEV V3 mulv(const M3& m, V3 v) { return col0(m) * v.x + col1(m) * v.y + col2(m) * v.z; }
// Mat3::transpose_mul_vec3 (lib.rs:270-273)
BH_DEV V3 tmulv(const M3& m, V3 v) { return v3(dot(col0(m), v), dot(col1(m), v), dot(col2(m), v)); }
// Mat3::mul_mat3 (lib.rs:275-282)
BH_DEV M3 mul(const M3& a, const M3& b) { return from_cols(mulv(a, col0(b)), mulv(a, col1(b)), mulv(a, col2(b))); }
// Mat3::mul_diag (lib.rs:284-291)
BH_DEV M3 mul_diag(const M3& m, V3 s) { return from_cols(col0(m) * s.x, col1(m) * s.y, col2(m) * s.z); }
// Mat3::outer_product_self (lib.rs:305-318)
BH_DEV S3 outer_self(const M3& m) {
    V3 r0 = row0(m), r1 = row1(m), r2 = row2(m);
    return S3{dot(r0, r0), dot(r0, r1), dot(r0, r2), dot(r1, r1), dot(r1, r2), dot(r2, r2)};
}
// Mat2x3::mul_vec3 / mul_mat3 / rows / gram_matrix (lib.rs:330-384)
BH_DEV V2 mulv(const M23& m, V3 v) { return m.c0 * v.x + m.c1 * v.y + m.c2 * v.z; }
BH_DEV M23 mul(const M23& m, const M3& n) { return M23{mulv(m, col0(n)), mulv(m, col1(n)), mulv(m, col2(n))}; }
BH_DEV V3 row0(const M23& m) { return v3(m.c0.x, m.c1.x, m.c2.x); }
BH_DEV V3 row1(const M23& m) { return v3(m.c0.y, m.c1.y, m.c2.y); }
BH_DEV S2 gram(const M23& m) {
    S2 s;
    s.c00 = m.c0.x * m.c0.x + m.c1.x * m.c1.x + m.c2.x * m.c2.x;
    s.c01 = m.c0.x * m.c0.y + m.c1.x * m.c1.y + m.c2.x * m.c2.y;
    s.c11 = m.c0.y * m.c0.y + m.c1.y * m.c1.y + m.c2.y * m.c2.y;
    return s;
}
// Sym2 (lib.rs:395-458)
BH_DEV V2 mulv(const S2& s, V2 v) { return v2(s.c00, s.c01) * v.x + v2(s.c01, s.c11) * v.y; }
BH_DEV M23 mul(const S2& s, const M23& n) { return M23{mulv(s, n.c0), mulv(s, n.c1), mulv(s, n.c2)}; }
BH_DEV S2 scale(const S2& s, float f) { return S2{s.c00 * f, s.c01 * f, s.c11 * f}; }
BH_DEV float max_abs(const S2& s) { return bh_maxf(bh_maxf(bh_absf(s.c00), bh_absf(s.c11)), bh_absf(s.c01)); }
BH_DEV S2 inverse(const S2& s) {
    float det = s.c00 * s.c11 - s.c01 * s.c01;
    bool inv = det > 0.0f;
    float inv_det = inv ? 1.0f / det : 0.0f;
    return S2{s.c11 * inv_det, -s.c01 * inv_det, s.c00 * inv_det};
}
BH_DEV float det_strict(const S2& s) {
    float ad = s.c00 * s.c11;
    float bc = s.c01 * s.c01;
    return ad - bc;
}
BH_DEV bool finite2(const S2& s) { return bh_is_finite(s.c00) && bh_is_finite(s.c11) && bh_is_finite(s.c01); }
// Mat2x3::transpose_congruence_sym2 (lib.rs:357-370)
BH_DEV S3 tcong(const M23& m, const S2& s) {
    V2 sc0 = mulv(s, m.c0), sc1 = mulv(s, m.c1), sc2 = mulv(s, m.c2);
    return S3{dot(m.c0, sc0), dot(m.c0, sc1), dot(m.c0, sc2), dot(m.c1, sc1), dot(m.c1, sc2), dot(m.c2, sc2)};
}
// Sym3 (lib.rs:472-543)
BH_DEV V3 srow0(const S3& s) { return v3(s.c00, s.c01, s.c02); }
BH_DEV V3 srow1(const S3& s) { return v3(s.c01, s.c11, s.c12); }
BH_DEV V3 srow2(const S3& s) { return v3(s.c02, s.c12, s.c22); }
BH_DEV V3 mulv(const S3& s, V3 v) { return srow0(s) * v.x + srow1(s) * v.y + srow2(s) * v.z; }
BH_DEV S3 scale(const S3& s, float f) { return S3{s.c00 * f, s.c01 * f, s.c02 * f, s.c11 * f, s.c12 * f, s.c22 * f}; }
BH_DEV M3 mul(const S3& s, const M3& m) { return from_cols(mulv(s, col0(m)), mulv(s, col1(m)), mulv(s, col2(m))); }
BH_DEV S3 cong(const S3& s, const M3& m) {
    V3 sr0 = mulv(s, row0(m)), sr1 = mulv(s, row1(m)), sr2 = mulv(s, row2(m));
    return S3{dot(row0(m), sr0), dot(row0(m), sr1), dot(row0(m), sr2), dot(row1(m), sr1), dot(row1(m), sr2), dot(row2(m), sr2)};
}
BH_DEV S3 tcong(const S3& s, const M3& m) {
    V3 sc0 = mulv(s, col0(m)), sc1 = mulv(s, col1(m)), sc2 = mulv(s, col2(m));
    return S3{dot(col0(m), sc0), dot(col0(m), sc1), dot(col0(m), sc2), dot(col1(m), sc1), dot(col1(m), sc2), dot(col2(m), sc2)};
}

// ---- camera -----------------------------------------------------------------

BH_DEV M3 view_rot(const bh_project_uniforms& u) {
    const float* v = u.viewmat;
    return M3{v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7], v[8]};
}
// world_to_cam (kernels/helpers.rs:477-482)
BH_DEV V3 world_to_cam(const bh_project_uniforms& u, V3 mean) {
    return mulv(view_rot(u), mean) + v3(u.viewmat[9], u.viewmat[10], u.viewmat[11]);
}
// project_pinhole (camera_model/pinhole.rs:24-30)
BH_DEV V2 project_pinhole(const bh_project_uniforms& u, V3 p) {
    float inv_z = 1.0f / p.z;
    return v2(u.fx * p.x * inv_z + u.cx, u.fy * p.y * inv_z + u.cy);
}
// calculate_project_jacobian_pinhole (pinhole.rs:32-56)
BH_DEV M23 jacobian_pinhole(const bh_project_uniforms& u, V3 p) {
    float inv_z = 1.0f / p.z;
    float dx = u.fx * inv_z;
    float dy = u.fy * inv_z;
    float cxl = bh_clampf(p.x * inv_z, u.lim_neg_x, u.lim_pos_x);
    float cyl = bh_clampf(p.y * inv_z, u.lim_neg_y, u.lim_pos_y);
    return M23{v2(dx, 0.0f), v2(0.0f, dy), v2(-dx * cxl, -dy * cyl)};
}
// ---- camera models (kernels/camera_model/*.rs) --------------------------------
// The model is a template parameter (the reference makes it a comptime
// parameter of every projection kernel); its coefficients come from
// u.camera_params in the reference's struct order.  Each function restates the
// reference's expression term by term, so both sides round alike.
enum : int { kCamPinhole = 0, kCamKB4 = 1, kCamRT8 = 2, kCamTPF = 3 };

// project_kb4 (kannala_brandt_4.rs:18-52); also the radial part of TPF
BH_DEV V2 project_kb4(const bh_project_uniforms& u, V3 p) {
    const float* k = u.camera_params;
    const float x = p.x, y = p.y, z = p.z;
    const float inv_z = 1.0f / z;
    const float pin_u = u.fx * x * inv_z + u.cx, pin_v = u.fy * y * inv_z + u.cy;
    const float r = sqrtf(x * x + y * y);
    const float theta = bh_atan2f(r, z);
    const float t2 = theta * theta, t4 = t2 * t2, t6 = t2 * t4, t8 = t4 * t4;
    const float d = theta * (1.0f + k[0] * t2 + k[1] * t4 + k[2] * t6 + k[3] * t8);
    const float inv_r = 1.0f / r;
    const float fish_u = u.fx * (d * x * inv_r) + u.cx, fish_v = u.fy * (d * y * inv_r) + u.cy;
    const bool near_axis = r < 1e-6f;
    return v2(near_axis ? pin_u : fish_u, near_axis ? pin_v : fish_v);
}

// calculate_project_jacobian_kb4 (kannala_brandt_4.rs:54-136): no clamp
BH_DEV M23 jacobian_kb4(const bh_project_uniforms& u, V3 p) {
    const float* k = u.camera_params;
    const float fx = u.fx, fy = u.fy;
    const float x = p.x, y = p.y, z = p.z;
    const float inv_z = 1.0f / z;
    const float x2 = x * x, y2 = y * y, xy = x * y;
    const float r2 = x2 + y2;
    const float r = sqrtf(r2);
    const float inv_r = 1.0f / r;
    const float inv_r3 = inv_r * inv_r * inv_r;
    const float rho2 = r2 + z * z;
    const float inv_rho2 = 1.0f / rho2;
    const float inv_rho2_r = inv_rho2 * inv_r;
    const float theta = bh_atan2f(r, z);
    const float t2 = theta * theta, t4 = t2 * t2, t6 = t4 * t2, t8 = t4 * t4;
    const float d = theta * (1.0f + k[0] * t2 + k[1] * t4 + k[2] * t6 + k[3] * t8);
    const float dd = 1.0f + 3.0f * k[0] * t2 + 5.0f * k[1] * t4 + 7.0f * k[2] * t6 + 9.0f * k[3] * t8;
    const float dth_dx = x * z * inv_rho2_r, dth_dy = y * z * inv_rho2_r, dth_dz = -r * inv_rho2;
    const float dd_dx = dd * dth_dx, dd_dy = dd * dth_dy, dd_dz = dd * dth_dz;
    const float xr = x * inv_r, dxr_dx = y2 * inv_r3, dxr_dy = -xy * inv_r3;
    const float du_dx = fx * (dd_dx * xr + d * dxr_dx);
    const float du_dy = fx * (dd_dy * xr + d * dxr_dy);
    const float du_dz = fx * (dd_dz * xr);
    const float yr = y * inv_r, dyr_dx = -xy * inv_r3, dyr_dy = x2 * inv_r3;
    const float dv_dx = fy * (dd_dx * yr + d * dyr_dx);
    const float dv_dy = fy * (dd_dy * yr + d * dyr_dy);
    const float dv_dz = fy * (dd_dz * yr);
    const bool near_axis = r < 1e-6f;
    const float pdx = fx * inv_z, pdy = fy * inv_z;
    const float p_du_dz = -pdx * x * inv_z, p_dv_dz = -pdy * y * inv_z;
    return M23{v2(near_axis ? pdx : du_dx, near_axis ? 0.0f : dv_dx),
               v2(near_axis ? 0.0f : du_dy, near_axis ? pdy : dv_dy),
               v2(near_axis ? p_du_dz : du_dz, near_axis ? p_dv_dz : dv_dz)};
}

// project_rt8 (radial_tangential_8.rs:24-69)
BH_DEV V2 project_rt8(const bh_project_uniforms& u, V3 p) {
    const float* k = u.camera_params;
    const float p1 = k[6], p2 = k[7];
    const float xn = p.x / p.z, yn = p.y / p.z;
    const float xn2 = xn * xn, yn2 = yn * yn;
    const float r2 = xn2 + yn2, r4 = r2 * r2, r6 = r4 * r2;
    const float d = (1.0f + k[0] * r2 + k[1] * r4 + k[2] * r6) / (1.0f + k[3] * r2 + k[4] * r4 + k[5] * r6);
    const float xy = xn * yn;
    const float xd = xn * d + 2.0f * p1 * xy + p2 * (r2 + 2.0f * xn2);
    const float yd = yn * d + 2.0f * p2 * xy + p1 * (r2 + 2.0f * yn2);
    return v2(u.fx * xd + u.cx, u.fy * yd + u.cy);
}

// calculate_project_jacobian_rt8 (radial_tangential_8.rs:71-146): evaluated at
// the clamped normalised coordinate like the pinhole Jacobian
BH_DEV M23 jacobian_rt8(const bh_project_uniforms& u, V3 p) {
    const float* k = u.camera_params;
    const float p1 = k[6], p2 = k[7];
    const float fx = u.fx, fy = u.fy;
    const float z = p.z;
    const float inv_z = 1.0f / z, inv_z2 = inv_z * inv_z;
    const float xn = bh_clampf(p.x * inv_z, u.lim_neg_x, u.lim_pos_x);
    const float yn = bh_clampf(p.y * inv_z, u.lim_neg_y, u.lim_pos_y);
    const float xc = xn * z, yc = yn * z;
    const float r2 = xn * xn + yn * yn, r4 = r2 * r2, r6 = r4 * r2;
    const float n_poly = 1.0f + k[0] * r2 + k[1] * r4 + k[2] * r6;
    const float dn_poly = 1.0f + k[3] * r2 + k[4] * r4 + k[5] * r6;
    const float np_poly = k[0] + 2.0f * k[1] * r2 + 3.0f * k[2] * r4;
    const float dnp_poly = k[3] + 2.0f * k[4] * r2 + 3.0f * k[5] * r4;
    const float inv_dn = 1.0f / dn_poly, inv_dn2 = inv_dn * inv_dn;
    const float rv = n_poly * inv_dn;
    const float rpv = (np_poly * dn_poly - n_poly * dnp_poly) * inv_dn2;
    const float d00 = rv + 2.0f * xn * xn * rpv + 2.0f * p1 * yn + 6.0f * p2 * xn;
    const float d01 = 2.0f * xn * yn * rpv + 2.0f * p1 * xn + 2.0f * p2 * yn;
    const float d10 = d01;
    const float d11 = rv + 2.0f * yn * yn * rpv + 6.0f * p1 * yn + 2.0f * p2 * xn;
    return M23{v2(fx * d00 * inv_z, fy * d10 * inv_z), v2(fx * d01 * inv_z, fy * d11 * inv_z),
               v2(-fx * (d00 * xc + d01 * yc) * inv_z2, -fy * (d10 * xc + d11 * yc) * inv_z2)};
}

// thin_prism_polys (thin_prism_fisheye.rs:37-63): N_u, N_v and their x, y
// derivatives in camera-space x, y (the model divides them by z^2)
struct PrismPolys {
    float nu, nv, dnu_dx, dnu_dy, dnv_dx, dnv_dy;
};
BH_DEV PrismPolys thin_prism_polys(const bh_project_uniforms& u, float x, float y) {
    const float p1 = u.camera_params[4], p2 = u.camera_params[5];
    const float sx1 = u.camera_params[6], sy1 = u.camera_params[7];
    const float x2 = x * x, y2 = y * y, xy = x * y, r2 = x2 + y2;
    PrismPolys o;
    o.nu = 2.0f * p1 * xy + p2 * (3.0f * x2 + y2) + sx1 * r2;
    o.nv = 2.0f * p2 * xy + p1 * (x2 + 3.0f * y2) + sy1 * r2;
    o.dnu_dx = 2.0f * (p1 * y + (3.0f * p2 + sx1) * x);
    o.dnu_dy = 2.0f * (p1 * x + (p2 + sx1) * y);
    o.dnv_dx = 2.0f * (p2 * y + (p1 + sy1) * x);
    o.dnv_dy = 2.0f * (p2 * x + (3.0f * p1 + sy1) * y);
    return o;
}

// project_tpf (thin_prism_fisheye.rs:65-81)
BH_DEV V2 project_tpf(const bh_project_uniforms& u, V3 p) {
    const V2 kb = project_kb4(u, p);
    const float inv_z = 1.0f / p.z, inv_z2 = inv_z * inv_z;
    const PrismPolys t = thin_prism_polys(u, p.x, p.y);
    return v2(kb.x + u.fx * t.nu * inv_z2, kb.y + u.fy * t.nv * inv_z2);
}

// calculate_project_jacobian_tpf (thin_prism_fisheye.rs:83-114)
BH_DEV M23 jacobian_tpf(const bh_project_uniforms& u, V3 p) {
    const M23 kb = jacobian_kb4(u, p);
    const float fx = u.fx, fy = u.fy;
    const float inv_z = 1.0f / p.z, inv_z2 = inv_z * inv_z, inv_z3 = inv_z2 * inv_z;
    const PrismPolys t = thin_prism_polys(u, p.x, p.y);
    const float add_du_dx = fx * t.dnu_dx * inv_z2, add_du_dy = fx * t.dnu_dy * inv_z2;
    const float add_du_dz = -2.0f * fx * t.nu * inv_z3;
    const float add_dv_dx = fy * t.dnv_dx * inv_z2, add_dv_dy = fy * t.dnv_dy * inv_z2;
    const float add_dv_dz = -2.0f * fy * t.nv * inv_z3;
    return M23{v2(kb.c0.x + add_du_dx, kb.c0.y + add_dv_dx), v2(kb.c1.x + add_du_dy, kb.c1.y + add_dv_dy),
               v2(kb.c2.x + add_du_dz, kb.c2.y + add_dv_dz)};
}

// project (camera_model/mod.rs:50-62)
template <int CAM>
BH_DEV V2 project_point(const bh_project_uniforms& u, V3 p) {
    if (CAM == kCamKB4) return project_kb4(u, p);
    if (CAM == kCamRT8) return project_rt8(u, p);
    if (CAM == kCamTPF) return project_tpf(u, p);
    return project_pinhole(u, p);
}

// calculate_project_jacobian (camera_model/mod.rs:64-80)
template <int CAM>
BH_DEV M23 jacobian(const bh_project_uniforms& u, V3 p) {
    if (CAM == kCamKB4) return jacobian_kb4(u, p);
    if (CAM == kCamRT8) return jacobian_rt8(u, p);
    if (CAM == kCamTPF) return jacobian_tpf(u, p);
    return jacobian_pinhole(u, p);
}

// The depth cull of project_forward (project_forward.rs:49-62): pinhole drops
// z < 0.01; the other models drop splats whose view angle exceeds
// half_max_render_fov.
template <int CAM>
BH_DEV bool depth_culled(const bh_project_uniforms& u, V3 mean_c) {
    if (CAM == kCamPinhole) return mean_c.z < 0.01f;
    const float r = sqrtf(mean_c.x * mean_c.x + mean_c.y * mean_c.y);
    return bh_atan2f(r, mean_c.z) > u.half_max_render_fov;
}

// calc_cov2d (kernels/helpers.rs:297-330)
template <int CAM>
BH_DEV S2 calc_cov2d(const bh_project_uniforms& u, V3 sc, Q4 q, V3 mean_c) {
    M3 ns = mul_diag(mul(view_rot(u), qmat(q)), sc);
    M23 jac = jacobian<CAM>(u, mean_c);
    S2 raw = gram(mul(jac, ns));
    const float lim = 1.0e18f;
    float ma = max_abs(raw);
    float down = ma > lim ? lim / ma : 1.0f;
    return scale(raw, down);
}
// compensate_cov2d (kernels/helpers.rs:332-350)
template <bool MIP>
BH_DEV S2 compensate_cov2d(const S2& c, float& comp) {
    const float blur = MIP ? 0.1f : 0.3f;
    S2 b{c.c00 + blur, c.c01, c.c11 + blur};
    comp = 1.0f;
    if (MIP) {
        float det_raw = bh_maxf(det_strict(c), 0.0f);
        float det_b = det_strict(b);
        comp = sqrtf(det_raw / det_b);
    }
    return b;
}
// compute_bbox_extent (kernels/helpers.rs:227-241)
BH_DEV V2 bbox_extent(const S2& conic, float pt) {
    float det = conic.c00 * conic.c11 - conic.c01 * conic.c01;
    bool degenerate = det <= 0.0f;
    float inv_det = degenerate ? 0.0f : 1.0f / det;
    float ex = sqrtf(2.0f * pt * conic.c11 * inv_det);
    float ey = sqrtf(2.0f * pt * conic.c00 * inv_det);
    return v2(degenerate ? -1.0f : ex, degenerate ? -1.0f : ey);
}
struct TileBox {
    uint32_t min_x, min_y, max_x, max_y;
};
// get_bbox / get_tile_bbox (kernels/helpers.rs:99-148) for 16 x TH tiles
// (TH = 16, or 8 for the rasterizer's 16x8 candidate tiles)
template <int TH = 16>
BH_DEV TileBox tile_bbox(V2 m, V2 e, uint32_t bw, uint32_t bh) {
    float cx = m.x / 16.0f, cy = m.y / (float)TH, dx = e.x / 16.0f, dy = e.y / (float)TH;
    float bwf = (float)bw, bhf = (float)bh;
    TileBox b;
    b.min_x = (uint32_t)bh_clampf(cx - dx, 0.0f, bwf);
    b.min_y = (uint32_t)bh_clampf(cy - dy, 0.0f, bhf);
    b.max_x = (uint32_t)bh_clampf(cx + dx + 1.0f, 0.0f, bwf);
    b.max_y = (uint32_t)bh_clampf(cy + dy + 1.0f, 0.0f, bhf);
    return b;
}
// calc_sigma (brush-cube/src/lib.rs:632-638)
BH_DEV float calc_sigma(float px, float py, const S2& c, float x, float y) {
    float dx = px - x;
    float dy = py - y;
    return 0.5f * (c.c00 * dx * dx + c.c11 * dy * dy) + c.c01 * dx * dy;
}
// will_primitive_contribute (kernels/helpers.rs:241-280) on the 16 x TH rect
// of tile (tx, ty) (tile_rect, helpers.rs:96-111)
template <int TH = 16>
BH_DEV bool will_contribute(uint32_t tx, uint32_t ty, V2 m, const S2& c, float pt) {
    float min_x = (float)(tx * 16u), min_y = (float)(ty * (uint32_t)TH);
    float max_x = min_x + 16.0f, max_y = min_y + (float)TH;
    bool x_left = m.x < min_x, x_right = m.x > max_x;
    bool in_x = !(x_left || x_right);
    bool y_above = m.y < min_y, y_below = m.y > max_y;
    bool in_y = !(y_above || y_below);
    bool hit = in_x && in_y;
    if (!hit) {
        float corner_x = x_left ? min_x : max_x;
        float corner_y = y_above ? min_y : max_y;
        float width = max_x - min_x;
        float height = max_y - min_y;
        float dxf = x_left ? width : -width;
        float dyf = y_above ? height : -height;
        float diff_x = m.x - corner_x;
        float diff_y = m.y - corner_y;
        // each quotient only matters off its own row/column: skip the
        // division where the reference's select discards it
        float tt_x = 0.0f, tt_y = 0.0f;
        if (!in_y) tt_x = bh_clampf((dxf * c.c00 * diff_x + dxf * c.c01 * diff_y) / (dxf * c.c00 * dxf), 0.0f, 1.0f);
        if (!in_x) tt_y = bh_clampf((dyf * c.c01 * diff_x + dyf * c.c11 * diff_y) / (dyf * c.c11 * dyf), 0.0f, 1.0f);
        float px = corner_x + tt_x * dxf;
        float py = corner_y + tt_y * dyf;
        hit = calc_sigma(px, py, c, m.x, m.y) <= pt;
    }
    return hit;
}

// ---- alpha cutoff (kernels/helpers.rs:161-190) --------------------------------
constexpr float kCutMid = 1.0f / 255.0f;
constexpr float kCutBand = 1.0e-3f;
BH_DEV float cutoff_weight(float alpha) {
    float t = bh_clampf((alpha - (kCutMid - 0.5f * kCutBand)) / kCutBand, 0.0f, 1.0f);
    return t * t * (3.0f - 2.0f * t);
}
BH_DEV float cutoff_weight_deriv(float alpha) {
    const float low = kCutMid - 0.5f * kCutBand;
    const float high = kCutMid + 0.5f * kCutBand;
    bool inside = alpha > low && alpha < high;
    float t = (alpha - low) / kCutBand;
    return inside ? (6.0f * t - 6.0f * t * t) / kCutBand : 0.0f;
}

// A colour channel as the blend kernels stage it: negative values become -0
// and -0 becomes +0, others stay.  Added into a non-negative sum it acts as
// max(c, 0) bit for bit, and its sign bit is the gradient gate of the
// reference (v_rgb only where c >= 0, rasterize_backwards.rs:330-338).
BH_DEV float staged_colour(float c) { return c < 0.0f ? -0.0f : c + 0.0f; }
BH_DEV bool colour_gate(float staged) { return (bh_as_uint(staged) >> 31) == 0u; }

// Largest sigma at which a splat of opacity `opac` can still pass the alpha
// cutoff, plus a margin.  For sigma above it, opac * exp(-sigma) rounds below
// the cutoff (1/255, or the lower edge of the smooth band) with certainty:
// exp and log are within 2 ulp and the margin of 1e-3 exceeds their combined
// relative error by three orders of magnitude.  Callers use it to skip the
// exp of pairs that cannot contribute; every pair that can is evaluated
// exactly as before.
template <bool SMOOTH>
BH_DEV float sigma_cutoff(float opac) {
    const float alpha_min = SMOOTH ? (kCutMid - 0.5f * kCutBand) : kCutMid;
    return bh_logf(opac / alpha_min) + 1.0e-3f;
}
// log2(e) in float: the blend kernels compare the power in base 2
// (bh_power_log2) with kLog2e * sigma_cutoff, whose margin of 1e-3 (1.4e-3 in
// base 2) still exceeds the rounding of the scaled conic, power and product
// by three orders of magnitude.
constexpr float kLog2e = 1.44269504088896340736f;

// Lower bound on the power 0.5 d^T C d (d = p - m) over the pixel centres of
// the rectangle [x0, x1] x [y0, y1]: 0 if m lies inside, otherwise the least
// of the four clamped edge minimisers (the power restricted to a horizontal
// edge is minimised at dx = -c01 dy / c00, to a vertical one at
// dy = -c01 dx / c11).  A splat whose bound exceeds its sigma_cutoff by more
// than the float error of evaluating the power (1e-5 of the largest term
// magnitude in the rectangle; the evaluation error is below 1e-6 of it) can
// contribute to no pixel of the rectangle.
BH_DEV bool may_touch_rect(float mx, float my, const S2& c, float cutoff, float x0, float y0, float x1, float y1) {
    if (mx >= x0 && mx <= x1 && my >= y0 && my <= y1) return true;
    float best = 3.0e38f;
    const float ey[2] = {y0, y1};
    const float ex[2] = {x0, x1};
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const float dy = ey[k] - my;
        const float dx = bh_clampf(mx - c.c01 * dy / c.c00, x0, x1) - mx;
        best = bh_minf(best, 0.5f * (c.c00 * dx * dx + c.c11 * dy * dy) + c.c01 * dx * dy);
    }
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const float dx = ex[k] - mx;
        const float dy = bh_clampf(my - c.c01 * dx / c.c11, y0, y1) - my;
        best = bh_minf(best, 0.5f * (c.c00 * dx * dx + c.c11 * dy * dy) + c.c01 * dx * dy);
    }
    const float mdx = bh_maxf(bh_absf(x0 - mx), bh_absf(x1 - mx));
    const float mdy = bh_maxf(bh_absf(y0 - my), bh_absf(y1 - my));
    const float mag = c.c00 * mdx * mdx + c.c11 * mdy * mdy + 2.0f * bh_absf(c.c01) * mdx * mdy;
    return !(best > cutoff + 1.0e-5f * mag + 1.0e-6f);
}

// 4-bit mask of the 16x4 pixel strips (tile rows 4k..4k+3) of the tile with
// pixel origin (ox, oy) that a splat may touch.
BH_DEV uint32_t strip_mask(float mx, float my, const S2& c, float cutoff, uint32_t ox, uint32_t oy) {
    uint32_t m = 0;
    const float x0 = (float)ox + 0.5f, x1 = (float)ox + 15.5f;
#pragma unroll
    for (uint32_t k = 0; k < 4; k++) {
        const float y0 = (float)(oy + 4u * k) + 0.5f;
        if (may_touch_rect(mx, my, c, cutoff, x0, y0, x1, y0 + 3.0f)) m |= 1u << k;
    }
    return m;
}

// ---- spherical harmonics (kernels/sh.rs) --------------------------------------
// Coefficient k of a splat's row, channel-interleaved: row[3k + ch].
BH_DEV V3 rd3(const float* c, int k) { return v3(c[3 * k], c[3 * k + 1], c[3 * k + 2]); }

// sh_coeffs_to_color (sh.rs:151-247); `c` points at the splat's SH row.
template <int DEG>
BH_DEV V3 sh_to_color(const float* c, V3 v) {
    V3 color = rd3(c, 0) * 0.2820948f;
    if (DEG >= 1) {
        const float f0a = 0.4886025f;
        color = color + rd3(c, 1) * (-f0a * v.y);
        color = color + rd3(c, 2) * (f0a * v.z);
        color = color + rd3(c, 3) * (-f0a * v.x);
        if (DEG >= 2) {
            float z2 = v.z * v.z;
            float f0b = -1.0925485f * v.z;
            const float f1a = 0.54627424f;
            float fc1 = v.x * v.x - v.y * v.y;
            float fs1 = 2.0f * v.x * v.y;
            float p4 = f1a * fs1, p5 = f0b * v.y, p6 = 0.9461747f * z2 - 0.31539157f;
            float p7 = f0b * v.x, p8 = f1a * fc1;
            color = color + rd3(c, 4) * p4;
            color = color + rd3(c, 5) * p5;
            color = color + rd3(c, 6) * p6;
            color = color + rd3(c, 7) * p7;
            color = color + rd3(c, 8) * p8;
            if (DEG >= 3) {
                float f0c = -2.285229f * z2 + 0.4570458f;
                float f1b = 1.4453057f * v.z;
                const float f2a = -0.5900436f;
                float fc2 = v.x * fc1 - v.y * fs1;
                float fs2 = v.x * fs1 + v.y * fc1;
                float p12 = v.z * (1.8658817f * z2 - 1.119529f);
                color = color + rd3(c, 9) * (f2a * fs2);
                color = color + rd3(c, 10) * (f1b * fs1);
                color = color + rd3(c, 11) * (f0c * v.y);
                color = color + rd3(c, 12) * p12;
                color = color + rd3(c, 13) * (f0c * v.x);
                color = color + rd3(c, 14) * (f1b * fc1);
                color = color + rd3(c, 15) * (f2a * fc2);
                if (DEG >= 4) {
                    float f0d = v.z * (-4.683326f * z2 + 2.0071396f);
                    float f1c = 3.3116114f * z2 - 0.47308735f;
                    float f2b = -1.7701308f * v.z;
                    const float f3a = 0.62583575f;
                    float fc3 = v.x * fc2 - v.y * fs2;
                    float fs3 = v.x * fs2 + v.y * fc2;
                    float p20 = 1.9843135f * v.z * p12 - 1.0062306f * p6;
                    color = color + rd3(c, 16) * (f3a * fs3);
                    color = color + rd3(c, 17) * (f2b * fs2);
                    color = color + rd3(c, 18) * (f1c * fs1);
                    color = color + rd3(c, 19) * (f0d * v.y);
                    color = color + rd3(c, 20) * p20;
                    color = color + rd3(c, 21) * (f0d * v.x);
                    color = color + rd3(c, 22) * (f1c * fc1);
                    color = color + rd3(c, 23) * (f2b * fc2);
                    color = color + rd3(c, 24) * (f3a * fc3);
                }
            }
        }
    }
    return color;
}

// Evaluate the SH basis functions (the factors of sh_coeffs_to_color_vjp,
// sh.rs:383-466) into basis[0..(DEG+1)^2).
template <int DEG>
BH_DEV void sh_basis(V3 v, float* basis) {
    basis[0] = 0.2820948f;
    if (DEG >= 1) {
        const float f0a = 0.4886025f;
        basis[1] = -f0a * v.y;
        basis[2] = f0a * v.z;
        basis[3] = -f0a * v.x;
        if (DEG >= 2) {
            float z2 = v.z * v.z;
            float f0b = -1.0925485f * v.z;
            const float f1a = 0.54627424f;
            float fc1 = v.x * v.x - v.y * v.y;
            float fs1 = 2.0f * v.x * v.y;
            float p6 = 0.9461747f * z2 - 0.31539157f;
            basis[4] = f1a * fs1;
            basis[5] = f0b * v.y;
            basis[6] = p6;
            basis[7] = f0b * v.x;
            basis[8] = f1a * fc1;
            if (DEG >= 3) {
                float f0c = -2.285229f * z2 + 0.4570458f;
                float f1b = 1.4453057f * v.z;
                const float f2a = -0.5900436f;
                float fc2 = v.x * fc1 - v.y * fs1;
                float fs2 = v.x * fs1 + v.y * fc1;
                float p12 = v.z * (1.8658817f * z2 - 1.119529f);
                basis[9] = f2a * fs2;
                basis[10] = f1b * fs1;
                basis[11] = f0c * v.y;
                basis[12] = p12;
                basis[13] = f0c * v.x;
                basis[14] = f1b * fc1;
                basis[15] = f2a * fc2;
                if (DEG >= 4) {
                    float f0d = v.z * (-4.683326f * z2 + 2.0071396f);
                    float f1c = 3.3116114f * z2 - 0.47308735f;
                    float f2b = -1.7701308f * v.z;
                    const float f3a = 0.62583575f;
                    float fc3 = v.x * fc2 - v.y * fs2;
                    float fs3 = v.x * fs2 + v.y * fc2;
                    basis[16] = f3a * fs3;
                    basis[17] = f2b * fs2;
                    basis[18] = f1c * fs1;
                    basis[19] = f0d * v.y;
                    basis[20] = 1.9843135f * v.z * p12 + -1.0062306f * p6;
                    basis[21] = f0d * v.x;
                    basis[22] = f1c * fc1;
                    basis[23] = f2b * fc2;
                    basis[24] = f3a * fc3;
                }
            }
        }
    }
}

// The z factor F(z) of the degree-l, order-m basis functions and dF/dz.
// Every basis function of sh_to_color above is F(z) times Re or Im of
// (x + i y)^m (cosine part at index l^2 + l + m, sine part at l^2 + l - m),
// with these F (the forward's constants; the m = 0 one of degree 4 is its
// recursion over degrees 3 and 2).
BH_DEV void sh_z_factor(int l, int m, float z, float& f, float& df) {
    const float z2 = z * z;
    switch (l * 8 + m) {
        case 8: f = 0.4886025f * z, df = 0.4886025f; break;
        case 9: f = -0.4886025f, df = 0.0f; break;
        case 16: f = 0.9461747f * z2 - 0.31539157f, df = 1.8923494f * z; break;
        case 17: f = -1.0925485f * z, df = -1.0925485f; break;
        case 18: f = 0.54627424f, df = 0.0f; break;
        case 24: f = z * (1.8658817f * z2 - 1.119529f), df = 5.5976451f * z2 - 1.119529f; break;
        case 25: f = -2.285229f * z2 + 0.4570458f, df = -4.570458f * z; break;
        case 26: f = 1.4453057f * z, df = 1.4453057f; break;
        case 27: f = -0.5900436f, df = 0.0f; break;
        case 32: {
            const float f3 = z * (1.8658817f * z2 - 1.119529f), d3 = 5.5976451f * z2 - 1.119529f;
            const float f2 = 0.9461747f * z2 - 0.31539157f, d2 = 1.8923494f * z;
            f = 1.9843135f * z * f3 - 1.0062306f * f2;
            df = 1.9843135f * (f3 + z * d3) - 1.0062306f * d2;
            break;
        }
        case 33: f = z * (-4.683326f * z2 + 2.0071396f), df = -14.049978f * z2 + 2.0071396f; break;
        case 34: f = 3.3116114f * z2 - 0.47308735f, df = 6.6232228f * z; break;
        case 35: f = -1.7701308f * z, df = -1.7701308f; break;
        default: f = 0.62583575f, df = 0.0f; break;  // l = m = 4
    }
}

// The colour's gradient with respect to the (unnormalised) view direction v
// for the upstream colour gradient vc: sum over basis functions of
// (c_k . vc) grad Y_k (sh_color_viewdir_vjp, sh.rs:249-381, computes the same
// derivative term by term).  With Y = F(z) P_m(x, y), P_m = Re or Im of
// (x + i y)^m: d/dx (x + i y)^m = m (x + i y)^(m-1) and d/dy = i m
// (x + i y)^(m-1), so a cosine/sine pair of order m with weights wc, ws adds
// F m (wc C + ws S, ws C - wc S) with C + i S = (x + i y)^(m-1) to the x and
// y components and F' (wc Re + ws Im)((x + i y)^m) to z.
template <int DEG>
BH_DEV V3 sh_viewdir_vjp(const float* c, V3 v, V3 vc) {
    // re[m] + i im[m] = (x + i y)^m
    float re[DEG + 1], im[DEG + 1];
    re[0] = 1.0f, im[0] = 0.0f;
#pragma unroll
    for (int m = 1; m <= DEG; m++) {
        re[m] = v.x * re[m - 1] - v.y * im[m - 1];
        im[m] = v.x * im[m - 1] + v.y * re[m - 1];
    }
    float gx = 0.0f, gy = 0.0f, gz = 0.0f;
#pragma unroll
    for (int l = 1; l <= DEG; l++) {
        const int k0 = l * l + l;
        float f, df;
        sh_z_factor(l, 0, v.z, f, df);
        gz += df * dot(rd3(c, k0), vc);
#pragma unroll
        for (int m = 1; m <= l; m++) {
            sh_z_factor(l, m, v.z, f, df);
            const float wc = dot(rd3(c, k0 + m), vc), ws = dot(rd3(c, k0 - m), vc);
            const float fm = f * (float)m;
            gx += fm * (wc * re[m - 1] + ws * im[m - 1]);
            gy += fm * (ws * re[m - 1] - wc * im[m - 1]);
            gz += df * (wc * re[m] + ws * im[m]);
        }
    }
    return v3(gx, gy, gz);
}

// ---- projection backward pieces (project_backwards.rs) -------------------------

// Gradient through q -> q / |q| (apply_normalize_vjp, project_backwards.rs:
// 19-52): the Jacobian (I - q q^T / |q|^2) / |q| applied to g, i.e.
// (|q|^2 g - (q . g) q) / |q|^3.
BH_DEV Q4 normalize_vjp(Q4 q, Q4 g) {
    const float n2 = qdot(q, q);
    const float qg = qdot(q, g);
    const float s = 1.0f / (sqrtf(n2) * n2);
    return Q4{(n2 * g.w - qg * q.w) * s, (n2 * g.x - qg * q.x) * s, (n2 * g.y - qg * q.y) * s,
              (n2 * g.z - qg * q.z) * s};
}
// Gradient of sum_ab V_ab R_ab(q) through the rotation matrix of a unit
// quaternion (quat_to_mat_vjp, project_backwards.rs:54-79).  The entries of R
// are 1 - 2(y^2 + z^2) on the diagonal and 2(xy -+ wz), 2(xz +- wy),
// 2(yz -+ wx) off it, so w meets only the antisymmetric part of V and each of
// x, y, z the symmetric part plus its own diagonal pair.  V is column-major
// (cI_R = V[R][I]).
BH_DEV Q4 quat_to_mat_vjp(Q4 q, const M3& v) {
    const float a_zy = v.c1z - v.c2y, a_xz = v.c2x - v.c0z, a_yx = v.c0y - v.c1x;  // V - V^T
    const float s_xy = v.c1x + v.c0y, s_xz = v.c2x + v.c0z, s_yz = v.c2y + v.c1z;  // V + V^T
    const float gw = q.x * a_zy + q.y * a_xz + q.z * a_yx;
    const float gx = q.w * a_zy + q.y * s_xy + q.z * s_xz - 2.0f * q.x * (v.c1y + v.c2z);
    const float gy = q.w * a_xz + q.x * s_xy + q.z * s_yz - 2.0f * q.y * (v.c0x + v.c2z);
    const float gz = q.w * a_yx + q.x * s_xz + q.y * s_yz - 2.0f * q.z * (v.c0x + v.c1y);
    return Q4{2.0f * gw, 2.0f * gx, 2.0f * gy, 2.0f * gz};
}
// Gradient through the inverse of a symmetric 2x2 matrix (inverse2x2_vjp,
// project_backwards.rs:81-99): with C = M^-1 (here `m`, the conic) and V the
// symmetric gradient with respect to C, dL/dM = -C V C, expanded entry by
// entry for C = [[a, b], [b, c]], V = [[p, q], [q, r]].
BH_DEV S2 inverse2x2_vjp(const S2& m, const S2& v) {
    const float a = m.c00, b = m.c01, c = m.c11, p = v.c00, q = v.c01, r = v.c11;
    const float ab = a * b, bc = b * c;
    return S2{-(a * a * p + 2.0f * ab * q + b * b * r), -(ab * p + (b * b + a * c) * q + bc * r),
              -(b * b * p + 2.0f * bc * q + c * c * r)};
}
// calculate_projection_vjp_pinhole (camera_model/pinhole.rs:58-123)
BH_DEV V3 projection_vjp_pinhole(const bh_project_uniforms& u, const M23& J, V3 mean_c, const S3& cov_c, const S2& v_cov2d,
                         V2 v_mean2d) {
    float fx = u.fx, fy = u.fy;
    float mx = mean_c.x, my = mean_c.y, mz = mean_c.z;
    float inv_z = 1.0f / mz;
    float mx_rz_raw = mx * inv_z, my_rz_raw = my * inv_z;
    float mx_rz = bh_clampf(mx_rz_raw, u.lim_neg_x, u.lim_pos_x);
    float my_rz = bh_clampf(my_rz_raw, u.lim_neg_y, u.lim_pos_y);
    bool in_x = mx_rz_raw <= u.lim_pos_x && mx_rz_raw >= u.lim_neg_x;
    bool in_y = my_rz_raw <= u.lim_pos_y && my_rz_raw >= u.lim_neg_y;
    float inv_z2 = inv_z * inv_z;
    float inv_z3 = inv_z2 * inv_z;
    float v_mx = fx * inv_z * v_mean2d.x;
    float v_my = fy * inv_z * v_mean2d.y;
    float v_mz = -(fx * mx * v_mean2d.x + fy * my * v_mean2d.y) * inv_z2;
    M23 tmp = mul(v_cov2d, J);
    float vj00 = 2.0f * dot(row0(tmp), srow0(cov_c));
    float vj11 = 2.0f * dot(row1(tmp), srow1(cov_c));
    float vj20 = 2.0f * dot(row0(tmp), srow2(cov_c));
    float vj21 = 2.0f * dot(row1(tmp), srow2(cov_c));
    float tx = mz * mx_rz;
    float ty = mz * my_rz;
    if (in_x)
        v_mx += -fx * inv_z2 * vj20;
    else
        v_mz += -fx * inv_z3 * vj20 * tx;
    if (in_y)
        v_my += -fy * inv_z2 * vj21;
    else
        v_mz += -fy * inv_z3 * vj21 * ty;
    v_mz += -fx * inv_z2 * vj00 - fy * inv_z2 * vj11 + 2.0f * fx * tx * inv_z3 * vj20 + 2.0f * fy * ty * inv_z3 * vj21;
    return v3(v_mx, v_my, v_mz);
}

// 2 (v_cov2d J) cov_c, the six entries (row u, row v) x (column 0..2)
struct VJ6 {
    float u0, u1, u2, v0, v1, v2;
};
BH_DEV VJ6 cov_jacobian_grad(const M23& J, const S3& cov_c, const S2& v_cov2d) {
    const M23 tmp = mul(v_cov2d, J);
    VJ6 o;
    o.u0 = 2.0f * dot(row0(tmp), srow0(cov_c));
    o.u1 = 2.0f * dot(row0(tmp), srow1(cov_c));
    o.u2 = 2.0f * dot(row0(tmp), srow2(cov_c));
    o.v0 = 2.0f * dot(row1(tmp), srow0(cov_c));
    o.v1 = 2.0f * dot(row1(tmp), srow1(cov_c));
    o.v2 = 2.0f * dot(row1(tmp), srow2(cov_c));
    return o;
}

// calculate_projection_vjp_kb4 (kannala_brandt_4.rs:138-337): J^T v_mean2d
// plus the contraction of 2 (v_cov2d J) cov_c with the second derivatives of
// the projection
BH_DEV V3 projection_vjp_kb4(const bh_project_uniforms& u, const M23& J, V3 mean_c, const S3& cov_c,
                             const S2& v_cov2d, V2 v_mean2d) {
    const float* k = u.camera_params;
    const float fx = u.fx, fy = u.fy;
    const float mx = mean_c.x, my = mean_c.y, mz = mean_c.z;
    const float r2 = mx * mx + my * my;
    const float r = bh_maxf(sqrtf(r2), 1.0e-8f);
    const float rho2 = r2 + mz * mz;
    const float theta = bh_atan2f(r, mz);
    const float th2 = theta * theta, th4 = th2 * th2, th6 = th4 * th2, th8 = th4 * th4;
    const float theta_d = theta * (1.0f + k[0] * th2 + k[1] * th4 + k[2] * th6 + k[3] * th8);
    const float p1 = 1.0f + 3.0f * k[0] * th2 + 5.0f * k[1] * th4 + 7.0f * k[2] * th6 + 9.0f * k[3] * th8;
    const float p2 = 6.0f * k[0] * theta + 20.0f * k[1] * theta * th2 + 42.0f * k[2] * theta * th4 +
                     72.0f * k[3] * theta * th6;
    const float inv_r = 1.0f / r;
    const float inv_r3 = inv_r * inv_r * inv_r;
    const float inv_r5 = inv_r3 * inv_r * inv_r;
    const float inv_rho2 = 1.0f / rho2;
    const float inv_rho2_sq = inv_rho2 * inv_rho2;
    const float inv_rho2_r = inv_rho2 * inv_r;
    const float dth_x = mx * mz * inv_rho2_r, dth_y = my * mz * inv_rho2_r, dth_z = -r * inv_rho2;
    const float xr = mx * inv_r, yr = my * inv_r;
    const float dxr_x = my * my * inv_r3, dxr_y = -mx * my * inv_r3;
    const float dyr_x = dxr_y, dyr_y = mx * mx * inv_r3;
    const float dg_x = p1 * dth_x, dg_y = p1 * dth_y, dg_z = p1 * dth_z;
    float v_mx = dot(v_mean2d, J.c0);
    float v_my = dot(v_mean2d, J.c1);
    float v_mz = dot(v_mean2d, J.c2);
    const VJ6 vj = cov_jacobian_grad(J, cov_c, v_cov2d);
    const float three_r2_z2 = 3.0f * r2 + mz * mz;
    const float r2_minus_z2 = r2 - mz * mz;
    const float h_th_00 = mz * (r2 * rho2 - mx * mx * three_r2_z2) * inv_r3 * inv_rho2_sq;
    const float h_th_11 = mz * (r2 * rho2 - my * my * three_r2_z2) * inv_r3 * inv_rho2_sq;
    const float h_th_01 = -mx * my * mz * three_r2_z2 * inv_r3 * inv_rho2_sq;
    const float h_th_02 = mx * r2_minus_z2 * inv_r * inv_rho2_sq;
    const float h_th_12 = my * r2_minus_z2 * inv_r * inv_rho2_sq;
    const float h_th_22 = 2.0f * mz * r * inv_rho2_sq;
    const float two_x2_my2 = 2.0f * mx * mx - my * my;
    const float two_y2_mx2 = 2.0f * my * my - mx * mx;
    const float h_xr_00 = -3.0f * mx * my * my * inv_r5;
    const float h_xr_01 = my * two_x2_my2 * inv_r5;
    const float h_xr_11 = mx * two_y2_mx2 * inv_r5;
    const float h_yr_00 = my * two_x2_my2 * inv_r5;
    const float h_yr_01 = mx * two_y2_mx2 * inv_r5;
    const float h_yr_11 = -3.0f * mx * mx * my * inv_r5;
    {  // (j, k) = (0, 0)
        const float d2g = p2 * dth_x * dth_x + p1 * h_th_00;
        const float d_ju = fx * (d2g * xr + dg_x * dxr_x + dg_x * dxr_x + theta_d * h_xr_00);
        const float d_jv = fy * (d2g * yr + dg_x * dyr_x + dg_x * dyr_x + theta_d * h_yr_00);
        v_mx += vj.u0 * d_ju + vj.v0 * d_jv;
    }
    {  // (1, 0)
        const float d2g = p2 * dth_y * dth_x + p1 * h_th_01;
        const float d_ju = fx * (d2g * xr + dg_y * dxr_x + dg_x * dxr_y + theta_d * h_xr_01);
        const float d_jv = fy * (d2g * yr + dg_y * dyr_x + dg_x * dyr_y + theta_d * h_yr_01);
        v_mx += vj.u1 * d_ju + vj.v1 * d_jv;
    }
    {  // (2, 0)
        const float d2g = p2 * dth_z * dth_x + p1 * h_th_02;
        const float d_ju = fx * (d2g * xr + dg_x * 0.0f + dg_z * dxr_x);
        const float d_jv = fy * (d2g * yr + dg_x * 0.0f + dg_z * dyr_x);
        v_mx += vj.u2 * d_ju + vj.v2 * d_jv;
    }
    {  // (0, 1)
        const float d2g = p2 * dth_x * dth_y + p1 * h_th_01;
        const float d_ju = fx * (d2g * xr + dg_x * dxr_y + dg_y * dxr_x + theta_d * h_xr_01);
        const float d_jv = fy * (d2g * yr + dg_x * dyr_y + dg_y * dyr_x + theta_d * h_yr_01);
        v_my += vj.u0 * d_ju + vj.v0 * d_jv;
    }
    {  // (1, 1)
        const float d2g = p2 * dth_y * dth_y + p1 * h_th_11;
        const float d_ju = fx * (d2g * xr + dg_y * dxr_y + dg_y * dxr_y + theta_d * h_xr_11);
        const float d_jv = fy * (d2g * yr + dg_y * dyr_y + dg_y * dyr_y + theta_d * h_yr_11);
        v_my += vj.u1 * d_ju + vj.v1 * d_jv;
    }
    {  // (2, 1)
        const float d2g = p2 * dth_z * dth_y + p1 * h_th_12;
        const float d_ju = fx * (d2g * xr + dg_y * 0.0f + dg_z * dxr_y);
        const float d_jv = fy * (d2g * yr + dg_y * 0.0f + dg_z * dyr_y);
        v_my += vj.u2 * d_ju + vj.v2 * d_jv;
    }
    {  // (0, 2)
        const float d2g = p2 * dth_x * dth_z + p1 * h_th_02;
        const float d_ju = fx * (d2g * xr + dg_z * dxr_x + dg_x * 0.0f);
        const float d_jv = fy * (d2g * yr + dg_z * dyr_x + dg_x * 0.0f);
        v_mz += vj.u0 * d_ju + vj.v0 * d_jv;
    }
    {  // (1, 2)
        const float d2g = p2 * dth_y * dth_z + p1 * h_th_12;
        const float d_ju = fx * (d2g * xr + dg_z * dxr_y + dg_y * 0.0f);
        const float d_jv = fy * (d2g * yr + dg_z * dyr_y + dg_y * 0.0f);
        v_mz += vj.u1 * d_ju + vj.v1 * d_jv;
    }
    {  // (2, 2)
        const float d2g = p2 * dth_z * dth_z + p1 * h_th_22;
        const float d_ju = fx * (d2g * xr);
        const float d_jv = fy * (d2g * yr);
        v_mz += vj.u2 * d_ju + vj.v2 * d_jv;
    }
    return v3(v_mx, v_my, v_mz);
}

// calculate_projection_vjp_rt8 (radial_tangential_8.rs:148-377): the Jacobian
// is routed through the clamp of the normalised coordinate (surrogate point)
BH_DEV V3 projection_vjp_rt8(const bh_project_uniforms& u, V3 mean_c, const S3& cov_c, const S2& v_cov2d,
                             V2 v_mean2d) {
    const float* k = u.camera_params;
    const float p1 = k[6], p2 = k[7];
    const float fx = u.fx, fy = u.fy;
    const float mx = mean_c.x, my = mean_c.y, mz = mean_c.z;
    const float inv_z = 1.0f / mz;
    const float mx_rz_raw = mx * inv_z, my_rz_raw = my * inv_z;
    const float mx_rz = bh_clampf(mx_rz_raw, u.lim_neg_x, u.lim_pos_x);
    const float my_rz = bh_clampf(my_rz_raw, u.lim_neg_y, u.lim_pos_y);
    const bool in_x = mx_rz_raw <= u.lim_pos_x && mx_rz_raw >= u.lim_neg_x;
    const bool in_y = my_rz_raw <= u.lim_pos_y && my_rz_raw >= u.lim_neg_y;
    const float xc = mx_rz * mz, yc = my_rz * mz;
    const float inv_z2 = inv_z * inv_z, inv_z3 = inv_z2 * inv_z;
    const float x = xc * inv_z, y = yc * inv_z;
    const float r2 = x * x + y * y, r4 = r2 * r2;
    const float n_poly = 1.0f + k[0] * r2 + k[1] * r4 + k[2] * r2 * r4;
    const float dn_poly = 1.0f + k[3] * r2 + k[4] * r4 + k[5] * r2 * r4;
    const float np_poly = k[0] + 2.0f * k[1] * r2 + 3.0f * k[2] * r4;
    const float dnp_poly = k[3] + 2.0f * k[4] * r2 + 3.0f * k[5] * r4;
    const float npp_poly = 2.0f * k[1] + 6.0f * k[2] * r2;
    const float dnpp_poly = 2.0f * k[4] + 6.0f * k[5] * r2;
    const float inv_dn = 1.0f / dn_poly, inv_dn2 = inv_dn * inv_dn, inv_dn3 = inv_dn2 * inv_dn;
    const float rr = n_poly * inv_dn;
    const float rrp = (np_poly * dn_poly - n_poly * dnp_poly) * inv_dn2;
    const float rrpp = (npp_poly * dn_poly * dn_poly - 2.0f * np_poly * dn_poly * dnp_poly -
                        n_poly * dnpp_poly * dn_poly + 2.0f * n_poly * dnp_poly * dnp_poly) *
                       inv_dn3;
    const float rx = 2.0f * x * rrp, ry = 2.0f * y * rrp;
    const float rpx = 2.0f * x * rrpp, rpy = 2.0f * y * rrpp;
    const float d00 = rr + 2.0f * x * x * rrp + 2.0f * p1 * y + 6.0f * p2 * x;
    const float d01 = 2.0f * x * y * rrp + 2.0f * p1 * x + 2.0f * p2 * y;
    const float d10 = d01;
    const float d11 = rr + 2.0f * y * y * rrp + 6.0f * p1 * y + 2.0f * p2 * x;
    const float js00 = fx * d00 * inv_z, js01 = fx * d01 * inv_z;
    const float js02 = -fx * (d00 * xc + d01 * yc) * inv_z2;
    const float js10 = fy * d10 * inv_z, js11 = fy * d11 * inv_z;
    const float js12 = -fy * (d10 * xc + d11 * yc) * inv_z2;
    const float je00 = in_x ? js00 : 0.0f, je10 = in_x ? js10 : 0.0f;
    const float je01 = in_y ? js01 : 0.0f, je11 = in_y ? js11 : 0.0f;
    const float je02 = (in_x ? 0.0f : mx_rz * js00) + (in_y ? 0.0f : my_rz * js01) + js02;
    const float je12 = (in_x ? 0.0f : mx_rz * js10) + (in_y ? 0.0f : my_rz * js11) + js12;
    float v_mx = je00 * v_mean2d.x + je10 * v_mean2d.y;
    float v_my = je01 * v_mean2d.x + je11 * v_mean2d.y;
    float v_mz = je02 * v_mean2d.x + je12 * v_mean2d.y;
    const VJ6 ve = cov_jacobian_grad(M23{v2(je00, je10), v2(je01, je11), v2(je02, je12)}, cov_c, v_cov2d);
    const float vs_u0 = in_x ? ve.u0 : mx_rz * ve.u2, vs_v0 = in_x ? ve.v0 : mx_rz * ve.v2;
    const float vs_u1 = in_y ? ve.u1 : my_rz * ve.u2, vs_v1 = in_y ? ve.v1 : my_rz * ve.v2;
    const float vs_u2 = ve.u2, vs_v2 = ve.v2;
    const float dd00_dx = rx + 4.0f * x * rrp + 2.0f * x * x * rpx + 6.0f * p2;
    const float dd00_dy = ry + 2.0f * x * x * rpy + 2.0f * p1;
    const float dd01_dx = 2.0f * y * rrp + 2.0f * x * y * rpx + 2.0f * p1;
    const float dd01_dy = 2.0f * x * rrp + 2.0f * x * y * rpy + 2.0f * p2;
    const float dd10_dx = dd01_dx, dd10_dy = dd01_dy;
    const float dd11_dx = rx + 2.0f * y * y * rpx + 2.0f * p2;
    const float dd11_dy = ry + 4.0f * y * rrp + 2.0f * y * y * rpy + 6.0f * p1;
    const float dd00_dxc = dd00_dx * inv_z, dd00_dyc = dd00_dy * inv_z;
    const float dd00_dz = -(xc * dd00_dx + yc * dd00_dy) * inv_z2;
    const float dd01_dxc = dd01_dx * inv_z, dd01_dyc = dd01_dy * inv_z;
    const float dd01_dz = -(xc * dd01_dx + yc * dd01_dy) * inv_z2;
    const float dd10_dxc = dd10_dx * inv_z, dd10_dyc = dd10_dy * inv_z;
    const float dd10_dz = -(xc * dd10_dx + yc * dd10_dy) * inv_z2;
    const float dd11_dxc = dd11_dx * inv_z, dd11_dyc = dd11_dy * inv_z;
    const float dd11_dz = -(xc * dd11_dx + yc * dd11_dy) * inv_z2;
    const float djs00_dxc = fx * dd00_dxc * inv_z, djs00_dyc = fx * dd00_dyc * inv_z;
    const float djs00_dz = fx * (dd00_dz * inv_z - d00 * inv_z2);
    const float djs01_dxc = fx * dd01_dxc * inv_z, djs01_dyc = fx * dd01_dyc * inv_z;
    const float djs01_dz = fx * (dd01_dz * inv_z - d01 * inv_z2);
    const float djs10_dxc = fy * dd10_dxc * inv_z, djs10_dyc = fy * dd10_dyc * inv_z;
    const float djs10_dz = fy * (dd10_dz * inv_z - d10 * inv_z2);
    const float djs11_dxc = fy * dd11_dxc * inv_z, djs11_dyc = fy * dd11_dyc * inv_z;
    const float djs11_dz = fy * (dd11_dz * inv_z - d11 * inv_z2);
    const float djs02_dxc = -fx * (dd00_dxc * xc + d00 + dd01_dxc * yc) * inv_z2;
    const float djs02_dyc = -fx * (dd00_dyc * xc + dd01_dyc * yc + d01) * inv_z2;
    const float djs02_dz = -fx * ((dd00_dz * xc + dd01_dz * yc) * inv_z2 - 2.0f * (d00 * xc + d01 * yc) * inv_z3);
    const float djs12_dxc = -fy * (dd10_dxc * xc + d10 + dd11_dxc * yc) * inv_z2;
    const float djs12_dyc = -fy * (dd10_dyc * xc + dd11_dyc * yc + d11) * inv_z2;
    const float djs12_dz = -fy * ((dd10_dz * xc + dd11_dz * yc) * inv_z2 - 2.0f * (d10 * xc + d11 * yc) * inv_z3);
    const float c_xc = vs_u0 * djs00_dxc + vs_u1 * djs01_dxc + vs_u2 * djs02_dxc + vs_v0 * djs10_dxc +
                       vs_v1 * djs11_dxc + vs_v2 * djs12_dxc;
    const float c_yc = vs_u0 * djs00_dyc + vs_u1 * djs01_dyc + vs_u2 * djs02_dyc + vs_v0 * djs10_dyc +
                       vs_v1 * djs11_dyc + vs_v2 * djs12_dyc;
    const float c_z = vs_u0 * djs00_dz + vs_u1 * djs01_dz + vs_u2 * djs02_dz + vs_v0 * djs10_dz +
                      vs_v1 * djs11_dz + vs_v2 * djs12_dz;
    if (in_x) v_mx += c_xc;
    if (in_y) v_my += c_yc;
    v_mz += c_z;
    if (!in_x) v_mz += mx_rz * c_xc;
    if (!in_y) v_mz += my_rz * c_yc;
    return v3(v_mx, v_my, v_mz);
}

// calculate_projection_vjp_tpf (thin_prism_fisheye.rs:116-203): the KB4 VJP
// with the full Jacobian plus the tangential / thin-prism Hessian terms
BH_DEV V3 projection_vjp_tpf(const bh_project_uniforms& u, const M23& J, V3 mean_c, const S3& cov_c,
                             const S2& v_cov2d, V2 v_mean2d) {
    const V3 kb = projection_vjp_kb4(u, J, mean_c, cov_c, v_cov2d, v_mean2d);
    const float p1 = u.camera_params[4], p2 = u.camera_params[5];
    const float sx1 = u.camera_params[6], sy1 = u.camera_params[7];
    const float fx = u.fx, fy = u.fy;
    const float inv_z = 1.0f / mean_c.z;
    const float inv_z2 = inv_z * inv_z, inv_z3 = inv_z2 * inv_z, inv_z4 = inv_z2 * inv_z2;
    const PrismPolys t = thin_prism_polys(u, mean_c.x, mean_c.y);
    const float d2nu_dxx = 6.0f * p2 + 2.0f * sx1, d2nu_dyy = 2.0f * p2 + 2.0f * sx1, d2nu_dxy = 2.0f * p1;
    const float d2nv_dxx = 2.0f * p1 + 2.0f * sy1, d2nv_dyy = 6.0f * p1 + 2.0f * sy1, d2nv_dxy = 2.0f * p2;
    const float h_u_00 = d2nu_dxx * inv_z2, h_u_01 = d2nu_dxy * inv_z2, h_u_11 = d2nu_dyy * inv_z2;
    const float h_u_02 = -2.0f * t.dnu_dx * inv_z3, h_u_12 = -2.0f * t.dnu_dy * inv_z3;
    const float h_u_22 = 6.0f * t.nu * inv_z4;
    const float h_v_00 = d2nv_dxx * inv_z2, h_v_01 = d2nv_dxy * inv_z2, h_v_11 = d2nv_dyy * inv_z2;
    const float h_v_02 = -2.0f * t.dnv_dx * inv_z3, h_v_12 = -2.0f * t.dnv_dy * inv_z3;
    const float h_v_22 = 6.0f * t.nv * inv_z4;
    const VJ6 vj = cov_jacobian_grad(J, cov_c, v_cov2d);
    const float v_mx = fx * (vj.u0 * h_u_00 + vj.u1 * h_u_01 + vj.u2 * h_u_02) +
                       fy * (vj.v0 * h_v_00 + vj.v1 * h_v_01 + vj.v2 * h_v_02);
    const float v_my = fx * (vj.u0 * h_u_01 + vj.u1 * h_u_11 + vj.u2 * h_u_12) +
                       fy * (vj.v0 * h_v_01 + vj.v1 * h_v_11 + vj.v2 * h_v_12);
    const float v_mz = fx * (vj.u0 * h_u_02 + vj.u1 * h_u_12 + vj.u2 * h_u_22) +
                       fy * (vj.v0 * h_v_02 + vj.v1 * h_v_12 + vj.v2 * h_v_22);
    return v3(kb.x + v_mx, kb.y + v_my, kb.z + v_mz);
}

// calculate_projection_vjp (camera_model/mod.rs:82-126)
template <int CAM>
BH_DEV V3 projection_vjp(const bh_project_uniforms& u, const M23& J, V3 mean_c, const S3& cov_c, const S2& v_cov2d,
                         V2 v_mean2d) {
    if (CAM == kCamKB4) return projection_vjp_kb4(u, J, mean_c, cov_c, v_cov2d, v_mean2d);
    if (CAM == kCamRT8) return projection_vjp_rt8(u, mean_c, cov_c, v_cov2d, v_mean2d);
    if (CAM == kCamTPF) return projection_vjp_tpf(u, J, mean_c, cov_c, v_cov2d, v_mean2d);
    return projection_vjp_pinhole(u, J, mean_c, cov_c, v_cov2d, v_mean2d);
}

}  // namespace bh
