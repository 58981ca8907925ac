// Device-side building blocks for the gfx950 decoder kernels: fixed dimensions, the decode
// control block, fp16 helpers, q4/q8 code unpacking and wave64 cross-lane reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "icua_shared.h"

namespace icua {

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;

__device__ __forceinline__ uint32_t as_u32(float v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ float as_f32(uint32_t v) { return __builtin_bit_cast(float, v); }
__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ uint32_t h2_bits(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(f16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (f16)f); }

// a.x*b.x + a.y*b.y + c with fp32 accumulation (v_dot2c_f32_f16).
__device__ __forceinline__ float dot2(f16x2 a, f16x2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

// ------------------------------------------------------------------------------------------
// Code unpacking.
//
// q4: a dword holds eight codes q0..q7 at nibbles 0..7 (byte j = q[2j] | q[2j+1] << 4).
// Writing a nibble into mantissa bits 6..9 of an fp16 whose exponent field encodes 1.0 gives
// the exact value 1 + q/16.  One dword yields the pairs (q0,q4) (q1,q5) (q2,q6) (q3,q7).
// Per group: sum_k (s q_k + b) x_k = 16 s (sum_k (1 + q_k/16) x_k - X) + b X, X = sum_k x_k.
__device__ __forceinline__ void q4_unpack(uint32_t v, f16x2 out[4]) {
    out[0] = as_h2(((v << 6) & 0x03C003C0u) | 0x3C003C00u);
    out[1] = as_h2(((v << 2) & 0x03C003C0u) | 0x3C003C00u);
    out[2] = as_h2(((v >> 2) & 0x03C003C0u) | 0x3C003C00u);
    out[3] = as_h2(((v >> 6) & 0x03C003C0u) | 0x3C003C00u);
}

// q8: bytes b0..b3 of a dword are int8 codes.  Flipping the sign bit gives u = q + 128 and a
// byte permute places u under the fp16 exponent of 1024, giving the exact value 1152 + q.
// One dword yields the pairs (q0,q2) (q1,q3).  Per group: sum s q x = s (sum (1152+q) x - 1152 X).
__device__ __forceinline__ void q8_unpack(uint32_t v, f16x2 out[2]) {
    const uint32_t u = v ^ 0x80808080u;
    out[0] = as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x05020400u));
    out[1] = as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x05030401u));
}

// ------------------------------------------------------------------------------------------
// Cross-lane primitives (wave64).

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return as_f32((uint32_t)__builtin_amdgcn_update_dpp(0, (int)as_u32(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane i <-> 7-i within 8
constexpr int DPP_MIRROR = 0x140;      // lane i <-> 15-i within 16

// Lanes 0-31 receive a(l) + a(l+32); lanes 32-63 receive b(l-32) + b(l).
__device__ __forceinline__ float swap32_add(float a, float b) {
    auto r = __builtin_amdgcn_permlane32_swap(as_u32(a), as_u32(b), false, false);
    return as_f32(r[0]) + as_f32(r[1]);
}
// Lanes with bit 4 clear receive a(l) + a(l+16); lanes with bit 4 set receive b(l-16) + b(l).
__device__ __forceinline__ float swap16_add(float a, float b) {
    auto r = __builtin_amdgcn_permlane16_swap(as_u32(a), as_u32(b), false, false);
    return as_f32(r[0]) + as_f32(r[1]);
}

// Sum over the 16 lanes of each row of 16 (every lane gets the row sum).
__device__ __forceinline__ float sum16(float v) {
    v += dpp<DPP_MIRROR>(v);
    v += dpp<DPP_HALF_MIRROR>(v);
    v += dpp<DPP_XOR2>(v);
    v += dpp<DPP_XOR1>(v);
    return v;
}
// Sum over all 64 lanes (every lane gets the total).
__device__ __forceinline__ float wave_sum(float v) {
    v = sum16(v);
    v = swap16_add(v, v);
    v = swap32_add(v, v);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<DPP_MIRROR>(v));
    v = fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp<DPP_XOR2>(v));
    v = fmaxf(v, dpp<DPP_XOR1>(v));
    auto r = __builtin_amdgcn_permlane16_swap(as_u32(v), as_u32(v), false, false);
    v = fmaxf(as_f32(r[0]), as_f32(r[1]));
    auto q = __builtin_amdgcn_permlane32_swap(as_u32(v), as_u32(v), false, false);
    return fmaxf(as_f32(q[0]), as_f32(q[1]));
}

// Max / sum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (every lane gets the result).
__device__ __forceinline__ float max_x4(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(as_u32(v), as_u32(v), false, false);
    v = fmaxf(as_f32(r[0]), as_f32(r[1]));
    auto q = __builtin_amdgcn_permlane32_swap(as_u32(v), as_u32(v), false, false);
    return fmaxf(as_f32(q[0]), as_f32(q[1]));
}
__device__ __forceinline__ float sum_x4(float v) {
    const float s = swap16_add(v, v);
    return swap32_add(s, s);
}

// Per-head RMSNorm(128) + RoPE of one 128-vector by one wave: lane i owns the rotation pair
// (i, i + 64).
__device__ __forceinline__ void norm_rope_pair(float& a, float& b, const float* w, const float* cs, int lane) {
    const float ss = wave_sum(a * a + b * b);
    const float scale = 1.0f / sqrtf(ss / (float)HD + EPS);
    a = a * scale * w[lane];
    b = b * scale * w[lane + 64];
    const float c = cs[2 * lane], sn = cs[2 * lane + 1];
    const float a2 = a * c - b * sn;
    const float b2 = b * c + a * sn;
    a = a2;
    b = b2;
}

// Transposed reduction of R row partials held by every lane (R = 4 or 8).  Afterwards the
// total of row r is held by the lanes l with l / (64 / R) == r.
template <int R>
__device__ __forceinline__ float reduce_rows(const float* v, int lane) {
    static_assert(R == 4 || R == 8, "R");
    if constexpr (R == 8) {
        float t[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) t[i] = swap32_add(v[i], v[i + 4]);
        float u0 = swap16_add(t[0], t[2]);
        float u1 = swap16_add(t[1], t[3]);
        const bool b3 = lane & 8;
        float keep = b3 ? u1 : u0, send = b3 ? u0 : u1;
        float w = keep + dpp<DPP_MIRROR>(send);
        w += dpp<DPP_HALF_MIRROR>(w);
        w += dpp<DPP_XOR2>(w);
        w += dpp<DPP_XOR1>(w);
        return w;
    } else {
        float t0 = swap32_add(v[0], v[2]);
        float t1 = swap32_add(v[1], v[3]);
        float u = swap16_add(t0, t1);
        return sum16(u);
    }
}

// (value, index) argmax step: larger value wins, ties go to the lower index
// (Shaders.swift:1476-1488, 1509-1530).
__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}
template <int CTRL>
__device__ __forceinline__ void argmax_dpp(float& v, int& i) {
    argmax_merge(v, i, dpp<CTRL>(v), dpp_i<CTRL>(i));
}
// Every lane gets the wave's (value, index) argmax: a butterfly of DPP moves within rows of 16
// and two lane-swap steps across rows (no LDS round trips).  argmax_merge is symmetric, so the
// order in which a swap returns the two lanes' pairs does not matter.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
    argmax_dpp<DPP_XOR1>(v, i);
    argmax_dpp<DPP_XOR2>(v, i);
    argmax_dpp<DPP_HALF_MIRROR>(v, i);
    argmax_dpp<DPP_MIRROR>(v, i);
    auto rv = __builtin_amdgcn_permlane16_swap(as_u32(v), as_u32(v), false, false);
    auto ri = __builtin_amdgcn_permlane16_swap((uint32_t)i, (uint32_t)i, false, false);
    v = as_f32(rv[0]);
    i = (int)ri[0];
    argmax_merge(v, i, as_f32(rv[1]), (int)ri[1]);
    auto qv = __builtin_amdgcn_permlane32_swap(as_u32(v), as_u32(v), false, false);
    auto qi = __builtin_amdgcn_permlane32_swap((uint32_t)i, (uint32_t)i, false, false);
    v = as_f32(qv[0]);
    i = (int)qi[0];
    argmax_merge(v, i, as_f32(qv[1]), (int)qi[1]);
}

// ------------------------------------------------------------------------------------------
// One dequantised element (Shaders.swift:464-476 embed_at): q4 s*q + b, q8 s*q, f16 half;
// row-major .icua layout.
__device__ __forceinline__ float dequant_rowmajor(int fmt, const uint8_t* E, const uint8_t* Esb, size_t row, int i,
                                                  int K) {
    if (fmt == FMT_Q4) {
        const uint8_t b = E[row * (K / 2) + (i >> 1)];
        const float q = (float)((i & 1) ? (b >> 4) : (b & 15));
        const f16x2 sb = as_h2(((const uint32_t*)Esb)[row * (K / 64) + (i >> 6)]);
        return (float)sb.x * q + (float)sb.y;
    } else if (fmt == FMT_Q8) {
        const float s = h2f(((const uint16_t*)Esb)[row * (K / 32) + (i >> 5)]);
        return s * (float)(int8_t)E[row * K + i];
    }
    return h2f(((const uint16_t*)E)[row * K + i]);
}

// The same element read from the GEMV tile layout (gemv.hip repack_codes_kernel): lane
// l = r + 16 q of chunk c holds 16 bytes; scales stay row-major.
__device__ __forceinline__ float dequant_tiled(int fmt, const uint8_t* E, const uint8_t* Esb, size_t row, int k, int K) {
    const size_t rb = row / 16;
    const int r = (int)(row % 16);
    if (fmt == FMT_Q4) {
        const int nc = K / 128, c = k / 128, h = (k % 128) / 64, kk = k % 64, q = kk / 16, j = kk % 16;
        const int d = j / 8, jj = j % 8;
        const uint8_t b = E[((rb * nc + c) * 64 + r + 16 * q) * 16 + 8 * h + 4 * d + (jj % 4)];
        const float qv = (float)((jj / 4) ? (b >> 4) : (b & 15));
        const f16x2 sb = as_h2(((const uint32_t*)Esb)[row * (K / 64) + k / 64]);
        return (float)sb.x * qv + (float)sb.y;
    } else if (fmt == FMT_Q8) {
        const int nc = K / 64, c = k / 64, h = (k % 64) / 32, q = (k % 32) / 8, j = k % 8;
        const float s = h2f(((const uint16_t*)Esb)[row * (K / 32) + k / 32]);
        return s * (float)(int8_t)E[((rb * nc + c) * 64 + r + 16 * q) * 16 + 8 * h + j];
    }
    const int nc = K / 32, c = k / 32, q = (k % 32) / 8, j = k % 8;
    return h2f(((const uint16_t*)E)[((rb * nc + c) * 64 + r + 16 * q) * 8 + j]);
}

}  // namespace icua
