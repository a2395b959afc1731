// ply.hip — PLY vertex rows <-> the splat layout (crates/brush-serde).
//
// The host resolves a PLY header into a column table; these kernels do the
// per-row work that the reference's serde row visitor does on the CPU
// (import.rs:341-502 and 504-720, export.rs:83-178), moving the element's
// bytes once over HBM:
//
//   ply_decode_rows       standard vertex rows (any property types, either
//                         byte order, any row stride) -> transforms [n,10],
//                         sh [n,C,3], raw opacities [n].  A workgroup stages
//                         its rows' bytes in LDS (16-byte loads, four in
//                         flight per thread), then writes each output array
//                         as one contiguous sweep, every element gathered
//                         from LDS through its column descriptor.
//   ply_decode_compressed the SuperSplat layout: per splat four packed u32
//                         words dequantised against its chunk's ranges
//                         (quant.rs:1-71) plus optional u8 SH rows.
//   ply_encode_rows       the export layout, staged through LDS the other
//                         way: the splat arrays are read as contiguous
//                         blocks, the f32 rows written as one sweep.
//
// Arithmetic follows the reference's f32 expressions operation for operation
// (no contraction: the library is built with -ffp-contract=off and IEEE
// division / square root); inverse_sigmoid takes the library's reproducible
// logf.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "bh_internal.h"
#include "bh_math.h"

namespace bh {
namespace {

constexpr uint32_t kPlyThreads = 256;
constexpr uint32_t kPlyMaxCoeffs = 25;                       // SH degree 4
constexpr uint32_t kPlyMaxColumns = 11 + 3 * kPlyMaxCoeffs;  // 86
constexpr uint32_t kPlyLdsBudget = 16384;                    // bytes of staged rows per workgroup
constexpr uint32_t kPlyMaxRowBytes = 32768;
constexpr float kShC0 = 0.28209479177387814f;                // shaders.rs SH_C0
constexpr uint32_t kSplatsPerChunk = 256;                    // import.rs:513

struct PlyColumns {
    bh_ply_column c[kPlyMaxColumns];
};

__host__ __device__ inline uint32_t ply_type_bytes(uint32_t type) {
    switch (type) {
        case BH_PLY_I8:
        case BH_PLY_U8: return 1;
        case BH_PLY_I16:
        case BH_PLY_U16: return 2;
        case BH_PLY_I32:
        case BH_PLY_U32:
        case BH_PLY_F32: return 4;
        case BH_PLY_F64: return 8;
        default: return 0;
    }
}

// `bytes` bytes at LDS byte address `a`, assembled little-endian, then
// byte-reversed for a big-endian file.
__device__ inline uint64_t lds_read(const uint8_t* lds, uint32_t a, uint32_t bytes, bool big) {
    uint64_t v = 0;
    if ((a & 3u) == 0u && bytes >= 4u) {
        const uint32_t* w = reinterpret_cast<const uint32_t*>(lds + a);
        v = w[0];
        if (bytes == 8u) v |= (uint64_t)w[1] << 32;
    } else {
        for (uint32_t i = 0; i < bytes; i++) v |= (uint64_t)lds[a + i] << (8u * i);
    }
    if (big) {
        if (bytes == 2u) v = __builtin_bswap16((uint16_t)v);
        else if (bytes == 4u) v = __builtin_bswap32((uint32_t)v);
        else if (bytes == 8u) v = __builtin_bswap64(v);
    }
    return v;
}

// Rust `as f32` of each PLY scalar type (serde's f32 visitor casts).
__device__ inline float ply_to_f32(uint64_t raw, uint32_t type) {
    switch (type) {
        case BH_PLY_I8: return (float)(int8_t)(uint8_t)raw;
        case BH_PLY_U8: return (float)(uint32_t)(uint8_t)raw;
        case BH_PLY_I16: return (float)(int16_t)(uint16_t)raw;
        case BH_PLY_U16: return (float)(uint32_t)(uint16_t)raw;
        case BH_PLY_I32: return (float)(int32_t)(uint32_t)raw;
        case BH_PLY_U32: return (float)(uint32_t)raw;
        case BH_PLY_F32: return bh_as_float((uint32_t)raw);
        default: {
            double d;
            __builtin_memcpy(&d, &raw, sizeof(d));
            return (float)d;
        }
    }
}

// ply_gaussian.rs:35-56 (de_quant) then sh.rs:20-31 (rgb_to_sh).
__device__ inline float ply_color_to_sh(uint64_t raw, uint32_t type) {
    float c;
    if (type == BH_PLY_U8) c = (float)(uint32_t)(uint8_t)raw / 255.0f;
    else if (type == BH_PLY_U16) c = (float)(uint32_t)(uint16_t)raw / 65535.0f;
    else c = bh_as_float((uint32_t)raw);
    return (c - 0.5f) / kShC0;
}

__device__ inline float ply_fetch(const uint8_t* lds, uint32_t slot_base, const bh_ply_column& col, bool big) {
    if (col.type == BH_PLY_CONST) return col.konst;
    const uint64_t raw = lds_read(lds, slot_base + col.offset, ply_type_bytes(col.type), big);
    return col.op == BH_PLY_OP_COLOR ? ply_color_to_sh(raw, col.type) : ply_to_f32(raw, col.type);
}

// Stages the bytes of output rows [r0, r0 + nr) in LDS and returns, through
// s_base, the LDS byte address of each row.  CONTIG (subsample 1, 16-byte
// aligned source): the rows are one span of memory, loaded as 16-byte words
// from floor16(r0 * R) on, four in flight per thread.  Otherwise each row
// r * subsample gets its own slot of slot_dwords dwords from floor4(start) on
// (slot_dwords * 4 >= R + 3 covers the shift).  Loads past src_bytes read 0.
template <bool CONTIG>
__device__ inline void stage_rows(uint32_t* s_stage, uint32_t* s_base, const uint8_t* __restrict__ src,
                                  uint64_t src_bytes, uint32_t row_bytes, uint64_t r0, uint32_t nr,
                                  uint32_t subsample, uint32_t slot_dwords) {
    if (CONTIG) {
        const uint64_t b0 = r0 * row_bytes;
        const uint64_t lo = b0 >> 4;
        const uint32_t n4 = (uint32_t)(((b0 + (uint64_t)nr * row_bytes + 15u) >> 4) - lo);
        const uint4* g4 = reinterpret_cast<const uint4*>(src) + lo;
        uint4* l4 = reinterpret_cast<uint4*>(s_stage);
        if ((lo + n4) * 16u <= src_bytes) {  // uniform: the span lies inside the buffer
            for (uint32_t i0 = threadIdx.x; i0 < n4; i0 += 4u * kPlyThreads) {
                // out-of-range slots redo word i0 (same value, same place): no
                // branches, so the four loads overlap
                const uint32_t i1 = i0 + kPlyThreads < n4 ? i0 + kPlyThreads : i0;
                const uint32_t i2 = i0 + 2u * kPlyThreads < n4 ? i0 + 2u * kPlyThreads : i0;
                const uint32_t i3 = i0 + 3u * kPlyThreads < n4 ? i0 + 3u * kPlyThreads : i0;
                const uint4 v0 = g4[i0];
                const uint4 v1 = g4[i1];
                const uint4 v2 = g4[i2];
                const uint4 v3 = g4[i3];
                l4[i0] = v0;
                l4[i1] = v1;
                l4[i2] = v2;
                l4[i3] = v3;
            }
        } else {  // the span's last word runs past the buffer: dword loads, zero beyond
            const uint32_t* g1 = reinterpret_cast<const uint32_t*>(src) + lo * 4u;
            const uint64_t avail = src_bytes / 4u - lo * 4u;
            uint32_t* l1 = s_stage;
            for (uint32_t i = threadIdx.x; i < n4 * 4u; i += kPlyThreads) l1[i] = i < avail ? g1[i] : 0u;
        }
        for (uint32_t r = threadIdx.x; r < nr; r += kPlyThreads) s_base[r] = (uint32_t)(b0 & 15u) + r * row_bytes;
    } else {
        const uint64_t stride = (uint64_t)subsample * row_bytes;
        const uint32_t* g1 = reinterpret_cast<const uint32_t*>(src);
        const uint64_t src_dwords = src_bytes / 4u;
        const uint32_t total = nr * slot_dwords;
        for (uint32_t base = threadIdx.x; base < total; base += 4u * kPlyThreads) {
            uint32_t v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t t = base + u * kPlyThreads;
                const uint32_t r = t / slot_dwords;
                const uint64_t dw = (((r0 + r) * stride) >> 2) + (t - r * slot_dwords);
                const bool ok = t < total && dw < src_dwords;
                const uint32_t w = g1[ok ? dw : 0u];  // dword 0 exists: num_rows >= 1
                v[u] = ok ? w : 0u;
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t t = base + u * kPlyThreads;
                if (t < total) s_stage[t] = v[u];
            }
        }
        for (uint32_t r = threadIdx.x; r < nr; r += kPlyThreads)
            s_base[r] = r * slot_dwords * 4u + (uint32_t)(((r0 + r) * stride) & 3u);
    }
}

// One output value of row base `rb`.  F32: every non-constant column is a
// little-endian f32 at a 4-byte aligned LDS address (one LDS dword read).
template <bool F32>
__device__ inline float ply_value(const uint32_t* s_stage, uint32_t rb, const bh_ply_column& col, bool big) {
    if (F32) {  // branch-free: a constant column's offset is 0, inside the row
        const float v = bh_as_float(s_stage[(rb + col.offset) >> 2]);
        return col.type == BH_PLY_CONST ? col.konst : v;
    }
    if (col.type == BH_PLY_CONST) return col.konst;
    return ply_fetch(reinterpret_cast<const uint8_t*>(s_stage), rb, col, big);
}

// Output rows [r0, r0 + nr) come from input rows r * subsample.  After the
// rows are staged, each output array is written as one contiguous sweep:
// transforms [nr, 10], opacities [nr], sh [nr, NC, 3], element t of the
// sweep taking column (t mod width) of row t / width.
template <int NC, bool CONTIG, bool F32>
__global__ __launch_bounds__(kPlyThreads) void ply_decode_rows_kernel(
    const uint8_t* __restrict__ src, uint64_t src_bytes, uint32_t row_bytes, uint64_t n_out, uint32_t subsample,
    uint32_t big, uint32_t rows_per_group, uint32_t slot_dwords, PlyColumns cols, float* __restrict__ transforms,
    float* __restrict__ sh, float* __restrict__ opac) {
    extern __shared__ uint4 s_dyn[];
    uint32_t* s_stage = reinterpret_cast<uint32_t*>(s_dyn);
    constexpr uint32_t kCols = 11u + 3u * NC;
    constexpr uint32_t kSh = 3u * NC;
    __shared__ bh_ply_column s_cols[kCols];
    __shared__ uint32_t s_base[kPlyThreads];
    if (threadIdx.x < kCols) s_cols[threadIdx.x] = cols.c[threadIdx.x];
    const uint64_t r0 = (uint64_t)blockIdx.x * rows_per_group;
    const uint32_t nr = (uint32_t)min((uint64_t)rows_per_group, n_out - r0);
    stage_rows<CONTIG>(s_stage, s_base, src, src_bytes, row_bytes, r0, nr, subsample, slot_dwords);
    __syncthreads();
    const bool be = big != 0u;
#pragma unroll 4
    for (uint32_t t = threadIdx.x; t < nr * 10u; t += kPlyThreads) {
        const uint32_t r = t / 10u;
        transforms[r0 * 10u + t] = ply_value<F32>(s_stage, s_base[r], s_cols[t - r * 10u], be);
    }
    for (uint32_t t = threadIdx.x; t < nr; t += kPlyThreads)
        opac[r0 + t] = ply_value<F32>(s_stage, s_base[t], s_cols[10], be);
#pragma unroll 4
    for (uint32_t t = threadIdx.x; t < nr * kSh; t += kPlyThreads) {
        const uint32_t r = t / kSh;
        sh[r0 * kSh + t] = ply_value<F32>(s_stage, s_base[r], s_cols[11u + (t - r * kSh)], be);
    }
}

// A u32 at any byte address of a global buffer, in the file's byte order.
__device__ inline uint32_t load_u32(const uint8_t* p, uint64_t a, bool big) {
    uint32_t v;
    if ((a & 3u) == 0u) {
        v = *reinterpret_cast<const uint32_t*>(p + a);
    } else {
        v = (uint32_t)p[a] | ((uint32_t)p[a + 1] << 8) | ((uint32_t)p[a + 2] << 16) | ((uint32_t)p[a + 3] << 24);
    }
    return big ? __builtin_bswap32(v) : v;
}

// quant.rs:4-7
__device__ inline float unpack_unorm(uint32_t packed, uint32_t bits) {
    return (float)packed / (float)((1u << bits) - 1u);
}

// import.rs:537-555: raw * (max - min) + min
__device__ inline float lerp_range(float raw, float lo, float hi) { return raw * (hi - lo) + lo; }

__global__ __launch_bounds__(kPlyThreads) void ply_decode_compressed_kernel(
    const float* __restrict__ chunks, const uint8_t* __restrict__ vrows, const uint8_t* __restrict__ srows,
    uint64_t n_out, uint32_t subsample, uint32_t big, bh_ply_compressed_layout L, float* __restrict__ transforms,
    float* __restrict__ sh, float* __restrict__ opac) {
    const uint64_t i = (uint64_t)blockIdx.x * kPlyThreads + threadIdx.x;
    if (i >= n_out) return;
    const bool be = big != 0u;
    const uint64_t j = i * subsample;
    const uint64_t vb = j * L.vertex_row_bytes;
    const uint32_t pp = load_u32(vrows, vb + L.position_offset, be);
    const uint32_t ps = load_u32(vrows, vb + L.scale_offset, be);
    const uint32_t pr = load_u32(vrows, vb + L.rotation_offset, be);
    const uint32_t pc = load_u32(vrows, vb + L.color_offset, be);
    const float* q = chunks + (j / kSplatsPerChunk) * 18u;
    float* t = transforms + i * 10u;
    // quant.rs:9-19, then QuantMeta::mean / scale
    const float p3[3] = {unpack_unorm((pp >> 21) & 0x7FFu, 11), unpack_unorm((pp >> 11) & 0x3FFu, 10),
                         unpack_unorm(pp & 0x7FFu, 11)};
    const float s3[3] = {unpack_unorm((ps >> 21) & 0x7FFu, 11), unpack_unorm((ps >> 11) & 0x3FFu, 10),
                         unpack_unorm(ps & 0x7FFu, 11)};
#pragma unroll
    for (int k = 0; k < 3; k++) {
        t[k] = lerp_range(p3[k], q[2 * k], q[2 * k + 1]);
        t[7 + k] = lerp_range(s3[k], q[6 + 2 * k], q[7 + 2 * k]);
    }
    // quant.rs:37-71: the largest component's index, the other three as
    // 10-bit unorms scaled by 1/sqrt(2); stored w x y z
    const uint32_t largest = (pr >> 30) & 3u;
    const float norm = 0.5f * 1.41421353816986083984375f;
    const float a = (unpack_unorm((pr >> 20) & 0x3FFu, 10) - 0.5f) / norm;
    const float b = (unpack_unorm((pr >> 10) & 0x3FFu, 10) - 0.5f) / norm;
    const float c = (unpack_unorm(pr & 0x3FFu, 10) - 0.5f) / norm;
    const float big_c = sqrtf(1.0f - (a * a + b * b + c * c));
    const float vals[3] = {a, b, c};
    int ind = 0;
#pragma unroll
    for (uint32_t k = 0; k < 4; k++) {
        if (k == largest) {
            t[3 + k] = big_c;
        } else {
            t[3 + k] = ind == 0 ? vals[0] : (ind == 1 ? vals[1] : vals[2]);
            ind++;
        }
    }
    // quant.rs:20-35 (most significant byte first); opacity is stored
    // post-sigmoid, colour as RGB in the chunk's range
    const float rgba[4] = {unpack_unorm((pc >> 24) & 0xFFu, 8), unpack_unorm((pc >> 16) & 0xFFu, 8),
                           unpack_unorm((pc >> 8) & 0xFFu, 8), unpack_unorm(pc & 0xFFu, 8)};
    opac[i] = bh_logf(rgba[3] / (1.0f - rgba[3]));
    const uint32_t cpc = L.sh_rest_count / 3u;
    const uint32_t n3c = 3u * (1u + cpc);
    float* o = sh + i * n3c;
#pragma unroll
    for (int k = 0; k < 3; k++) o[k] = (lerp_range(rgba[k], q[12 + 2 * k], q[13 + 2 * k]) - 0.5f) / kShC0;
    if (cpc == 0u) return;
    // ply_gaussian.rs:99-105 and import.rs:132-143: rest coefficient c of
    // channel ch is f_rest_{ch * cpc + c}
    const uint8_t* srow = srows + j * L.sh_row_bytes;
    for (uint32_t cc = 0; cc < cpc; cc++) {
#pragma unroll
        for (uint32_t ch = 0; ch < 3u; ch++) {
            const uint8_t v = srow[L.sh_offsets[ch * cpc + cc]];
            o[3u * (cc + 1u) + ch] = ((float)(uint32_t)v / 255.0f - 0.5f) * 8.0f;
        }
    }
}

// export.rs:83-178.  Output row of F = 11 + 3C floats:
//   x y z | scale_0..2 | opacity | rot_0..3 / max(|q|, 1e-12) | f_dc_0..2 |
//   f_rest channel-major (channel ch, coefficient c >= 1 at 14 + ch (C-1) + c - 1)
// The group's splats are staged in LDS as three blocks (transforms
// [rpg,10] | opacities [rpg] | sh [rpg,3C]); a table maps each output column
// to its block offset and per-row stride, so the row sweep is one LDS read
// and one division per value (by the row's quaternion norm for rot_*, by 1
// otherwise, which is exact).
template <int NC>
__device__ inline uint32_t encode_source(uint32_t f, uint32_t rpg) {
    constexpr uint32_t kSh = 3u * NC;
    constexpr uint32_t rest = NC - 1u;
    uint32_t base, stride, rot = 0u;
    if (f < 3u) {
        base = f, stride = 10u;
    } else if (f < 6u) {
        base = 4u + f, stride = 10u;
    } else if (f == 6u) {
        base = rpg * 10u, stride = 1u;
    } else if (f < 11u) {
        base = f - 4u, stride = 10u, rot = 1u;
    } else if (f < 14u || rest == 0u) {
        base = rpg * 11u + (f - 11u), stride = kSh;
    } else {
        const uint32_t e = f - 14u;
        const uint32_t ch = e / rest;
        base = rpg * 11u + 3u * (1u + (e - ch * rest)) + ch, stride = kSh;
    }
    return base | (stride << 16) | (rot << 31);
}

template <int NC, bool VEC>
__global__ __launch_bounds__(kPlyThreads) void ply_encode_rows_kernel(const float* __restrict__ transforms,
                                                                      const float* __restrict__ sh,
                                                                      const float* __restrict__ opac, uint64_t n,
                                                                      uint32_t rows_per_group,
                                                                      float* __restrict__ rows) {
    extern __shared__ float4 s_dyn_f[];
    float* s_in = reinterpret_cast<float*>(s_dyn_f);
    constexpr uint32_t kSh = 3u * NC;
    constexpr uint32_t F = 11u + kSh;
    __shared__ uint32_t s_tab[F];
    __shared__ float s_rn[kPlyThreads];
    const uint32_t rpg = rows_per_group;
    const uint64_t r0 = (uint64_t)blockIdx.x * rpg;
    const uint32_t nr = (uint32_t)min((uint64_t)rpg, n - r0);
    if (threadIdx.x < F) s_tab[threadIdx.x] = encode_source<NC>(threadIdx.x, rpg);
    // one load loop over the three blocks: [0, a) transforms, [a, b) opacities, [b, c) sh
    const uint32_t a = nr * 10u, b = a + nr, c = b + nr * kSh;
    if (VEC && (nr & 3u) == 0u) {  // every block a whole number of 16-byte words
        const uint32_t a4 = a / 4u, b4 = b / 4u, c4 = c / 4u;
        const float4* gt = reinterpret_cast<const float4*>(transforms + r0 * 10u);
        const float4* go = reinterpret_cast<const float4*>(opac + r0);
        const float4* gs = reinterpret_cast<const float4*>(sh + r0 * kSh);
        float4* lt = reinterpret_cast<float4*>(s_in);
        float4* lo = reinterpret_cast<float4*>(s_in + rpg * 10u);
        float4* ls = reinterpret_cast<float4*>(s_in + rpg * 11u);
        for (uint32_t i0 = threadIdx.x; i0 < c4; i0 += 4u * kPlyThreads) {
            // out-of-range slots redo word i0: the same value to the same place,
            // which keeps the loop free of branches so the four loads overlap
            uint32_t off[4], blk[4];
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t i = i0 + u * kPlyThreads;
                const uint32_t j = i < c4 ? i : i0;
                blk[u] = (j >= a4 ? 1u : 0u) + (j >= b4 ? 1u : 0u);
                off[u] = j - (blk[u] == 2u ? b4 : (blk[u] == 1u ? a4 : 0u));
                const float4* g = blk[u] == 2u ? gs : (blk[u] == 1u ? go : gt);
                v[u] = g[off[u]];
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                float4* l = blk[u] == 2u ? ls : (blk[u] == 1u ? lo : lt);
                l[off[u]] = v[u];
            }
        }
    } else {
        for (uint32_t i = threadIdx.x; i < c; i += kPlyThreads) {
            float v;
            if (i < a) v = transforms[r0 * 10u + i];
            else if (i < b) v = opac[r0 + (i - a)];
            else v = sh[r0 * kSh + (i - b)];
            const uint32_t li = i < a ? i : (i < b ? rpg * 10u + (i - a) : rpg * 11u + (i - b));
            s_in[li] = v;
        }
    }
    __syncthreads();
    for (uint32_t r = threadIdx.x; r < nr; r += kPlyThreads) {
        const float* q = s_in + r * 10u + 3u;
        // ((q0 q0 + q1 q1) + q2 q2) + q3 q3; fmaxf drops a NaN like Rust's f32::max
        s_rn[r] = fmaxf(sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]), 1e-12f);
    }
    __syncthreads();
#pragma unroll 4
    for (uint32_t k = threadIdx.x; k < nr * F; k += kPlyThreads) {
        const uint32_t r = k / F;
        const uint32_t e = s_tab[k - r * F];
        const float v = s_in[(e & 0xFFFFu) + r * ((e >> 16) & 0x7FFFu)];
        rows[r0 * F + k] = v / ((e >> 31) ? s_rn[r] : 1.0f);
    }
}

}  // namespace

uint32_t ply_rows_per_group(uint32_t bytes_per_row) {
    return std::max<uint32_t>(1u, std::min<uint32_t>(kPlyThreads, kPlyLdsBudget / std::max<uint32_t>(1u, bytes_per_row)));
}

template <int NC, bool CONTIG, bool F32>
void launch_decode_variant(bh_ctx* ctx, uint32_t blocks, uint32_t lds, const uint8_t* rows, uint64_t rows_bytes,
                           uint32_t row_bytes, uint64_t n_out, uint32_t subsample, uint32_t big, uint32_t nr,
                           uint32_t slot_dwords, const PlyColumns& cols, float* transforms, float* sh, float* opac) {
    launch(ctx, ply_decode_rows_kernel<NC, CONTIG, F32>, dim3(blocks), dim3(kPlyThreads), lds, rows, rows_bytes,
           row_bytes, n_out, subsample, big, nr, slot_dwords, cols, transforms, sh, opac);
}

template <int NC>
void launch_decode_nc(bh_ctx* ctx, bool contig, bool f32, uint32_t blocks, uint32_t lds, const uint8_t* rows,
                      uint64_t rows_bytes, uint32_t row_bytes, uint64_t n_out, uint32_t subsample, uint32_t big,
                      uint32_t nr, uint32_t slot_dwords, const PlyColumns& cols, float* t, float* sh, float* o) {
    if (contig && f32)
        launch_decode_variant<NC, true, true>(ctx, blocks, lds, rows, rows_bytes, row_bytes, n_out, subsample, big, nr,
                                              slot_dwords, cols, t, sh, o);
    else if (contig)
        launch_decode_variant<NC, true, false>(ctx, blocks, lds, rows, rows_bytes, row_bytes, n_out, subsample, big,
                                               nr, slot_dwords, cols, t, sh, o);
    else if (f32)
        launch_decode_variant<NC, false, true>(ctx, blocks, lds, rows, rows_bytes, row_bytes, n_out, subsample, big,
                                               nr, slot_dwords, cols, t, sh, o);
    else
        launch_decode_variant<NC, false, false>(ctx, blocks, lds, rows, rows_bytes, row_bytes, n_out, subsample, big,
                                                nr, slot_dwords, cols, t, sh, o);
}

bh_status launch_ply_decode_rows(bh_ctx* ctx, const uint8_t* rows, uint64_t rows_bytes, uint32_t row_bytes,
                                 uint64_t n_out, uint32_t subsample, uint32_t flags, const bh_ply_column* columns,
                                 uint32_t num_coeffs, float* transforms, float* sh, float* opac) {
    if (!(num_coeffs == 1 || num_coeffs == 4 || num_coeffs == 9 || num_coeffs == 16 || num_coeffs == 25))
        return set_error(ctx, BH_ERR_INVALID_ARG, "ply: num_coeffs must be 1, 4, 9, 16 or 25");
    const bool big = (flags & BH_PLY_BIG_ENDIAN) != 0u;
    PlyColumns cols{};
    const uint32_t ncols = 11u + 3u * num_coeffs;
    bool f32 = !big && row_bytes % 4u == 0u;
    for (uint32_t k = 0; k < ncols; k++) {
        const bh_ply_column& c = columns[k];
        if (c.type != BH_PLY_CONST) {
            const uint32_t sz = ply_type_bytes(c.type);
            if (sz == 0) return set_error(ctx, BH_ERR_INVALID_ARG, "ply: unknown column type");
            if ((uint64_t)c.offset + sz > row_bytes)
                return set_error(ctx, BH_ERR_INVALID_ARG, "ply: column outside the row");
            if (c.op > BH_PLY_OP_COLOR) return set_error(ctx, BH_ERR_INVALID_ARG, "ply: unknown column op");
            if (c.op == BH_PLY_OP_COLOR && c.type != BH_PLY_U8 && c.type != BH_PLY_U16 && c.type != BH_PLY_F32)
                return set_error(ctx, BH_ERR_INVALID_ARG, "ply: colour columns are u8, u16 or f32");
            f32 = f32 && c.type == BH_PLY_F32 && c.op == BH_PLY_OP_PLAIN && c.offset % 4u == 0u;
        }
        cols.c[k] = c;
        if (c.type == BH_PLY_CONST) cols.c[k].offset = 0;  // the f32 path reads offset 0 of the row, then selects
    }
    if (row_bytes > kPlyMaxRowBytes) return set_error(ctx, BH_ERR_INVALID_ARG, "ply: vertex rows over 32 KiB");
    const bool contig = subsample == 1u && (reinterpret_cast<uintptr_t>(rows) & 15u) == 0u;
    const uint32_t slot_dwords = (row_bytes + 6u) / 4u;
    uint32_t nr, lds;
    if (contig) {
        nr = ply_rows_per_group(row_bytes);
        lds = (nr * row_bytes + 15u) / 16u * 16u + 32u;  // the span plus its 16-byte misalignment
    } else {
        nr = ply_rows_per_group(slot_dwords * 4u);
        lds = nr * slot_dwords * 4u;
    }
    const uint32_t blocks = div_up(n_out, nr);
    KernelTimer t(ctx, "ply_decode_rows");
#define BH_PLY_DECODE(NC)                                                                                           \
    launch_decode_nc<NC>(ctx, contig, f32, blocks, lds, rows, rows_bytes, row_bytes, n_out, subsample, big ? 1u : 0u, \
                         nr, slot_dwords, cols, transforms, sh, opac)
    switch (num_coeffs) {
        case 1: BH_PLY_DECODE(1); break;
        case 4: BH_PLY_DECODE(4); break;
        case 9: BH_PLY_DECODE(9); break;
        case 16: BH_PLY_DECODE(16); break;
        default: BH_PLY_DECODE(25); break;
    }
#undef BH_PLY_DECODE
    return check_launch(ctx, "ply_decode_rows");
}

bh_status launch_ply_decode_compressed(bh_ctx* ctx, const float* chunks, const uint8_t* vrows, const uint8_t* srows,
                                       uint64_t n_out, uint32_t subsample, uint32_t flags,
                                       const bh_ply_compressed_layout& L, float* transforms, float* sh, float* opac) {
    KernelTimer t(ctx, "ply_decode_compressed");
    launch(ctx, ply_decode_compressed_kernel, dim3(div_up(n_out, kPlyThreads)), dim3(kPlyThreads), 0u, chunks, vrows,
           srows, n_out, subsample, (flags & BH_PLY_BIG_ENDIAN) ? 1u : 0u, L, transforms, sh, opac);
    return check_launch(ctx, "ply_decode_compressed");
}

bh_status launch_ply_encode_rows(bh_ctx* ctx, const float* transforms, const float* sh, const float* opac, uint64_t n,
                                 uint32_t num_coeffs, float* rows) {
    if (!(num_coeffs == 1 || num_coeffs == 4 || num_coeffs == 9 || num_coeffs == 16 || num_coeffs == 25))
        return set_error(ctx, BH_ERR_INVALID_ARG, "ply: num_coeffs must be 1, 4, 9, 16 or 25");
    const uint32_t per_row = (11u + 3u * num_coeffs) * 4u;
    // a multiple of 4 rows keeps every staged block 16-byte aligned; the
    // table packs LDS offsets below 2^16 floats
    const uint32_t nr = std::max<uint32_t>(4u, ply_rows_per_group(per_row) / 4u * 4u);
    if ((uint64_t)nr * (per_row / 4u) >= 65536u) return set_error(ctx, BH_ERR_INTERNAL, "ply: encode group too large");
    const bool vec = ((reinterpret_cast<uintptr_t>(transforms) | reinterpret_cast<uintptr_t>(sh) |
                       reinterpret_cast<uintptr_t>(opac)) & 15u) == 0u;
    const uint32_t blocks = div_up(n, nr);
    const uint32_t lds = nr * per_row;
    KernelTimer t(ctx, "ply_encode_rows");
#define BH_PLY_ENCODE(NC)                                                                                            \
    if (vec)                                                                                                         \
        launch(ctx, ply_encode_rows_kernel<NC, true>, dim3(blocks), dim3(kPlyThreads), lds, transforms, sh, opac, n,   \
               nr, rows);                                                                                              \
    else                                                                                                             \
        launch(ctx, ply_encode_rows_kernel<NC, false>, dim3(blocks), dim3(kPlyThreads), lds, transforms, sh, opac, n,  \
               nr, rows)
    switch (num_coeffs) {
        case 1: BH_PLY_ENCODE(1); break;
        case 4: BH_PLY_ENCODE(4); break;
        case 9: BH_PLY_ENCODE(9); break;
        case 16: BH_PLY_ENCODE(16); break;
        default: BH_PLY_ENCODE(25); break;
    }
#undef BH_PLY_ENCODE
    return check_launch(ctx, "ply_encode_rows");
}

}  // namespace bh
