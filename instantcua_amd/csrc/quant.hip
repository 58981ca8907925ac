// Group-wise quantisers of the .icua converter on gfx950 (Sources/Engine/Convert.swift:214-320),
// bit-exact with the reference's float32 arithmetic: every multiply and add is rounded on its
// own (no contraction), sums run in index order, division is correctly rounded, `.rounded()` is
// roundf (half away from zero) and Float16(x) rounds to nearest even (v_cvt_f16_f32).
//
// q8 (quantizeQ8, 215-241): four elements per lane; the 8 lanes of a group find its maximum with
// shuffles (max is exact in any order), derive the scale and write their own codes.
// q4 (quantizeQ4Raw / quantGroup, 243-320): one lane per 64-group, the group in registers.  The
// lane runs the reference's 5 x 5 clip grid: codes and one least-squares refit of (s, b), fp16
// rounding of both, the squared error of the rounded pair; the first candidate of least error
// wins.  The reference's second refit iteration only recomputes codes that the error pass
// overwrites, so it is not run.  When no candidate is accepted (every fp16 scale rounds to 0) the
// reference leaves the codes of the chunk's previous group in its code array; a second kernel
// copies them, so the output bytes match as well (the dequantised values are 0 either way).
#include <mutex>

#include "icua_device.h"
#include "icua_kernels.h"

namespace icua {
namespace {

// Swift's min / max on Float: min(x, y) = y < x ? y : x, max(x, y) = y >= x ? y : x.
__device__ __forceinline__ float sw_min(float x, float y) { return y < x ? y : x; }
__device__ __forceinline__ float sw_max(float x, float y) { return y >= x ? y : x; }

constexpr int QT = 256;  // threads per workgroup

__global__ __launch_bounds__(QT) void quant_q8_kernel(const float* __restrict__ m, int64_t n, int8_t* __restrict__ codes,
                                                      uint16_t* __restrict__ scales) {
#pragma clang fp contract(off)
    // Four consecutive elements per lane (one 16-byte load); group i / 32 = 8 lanes.
    const int64_t i4 = ((int64_t)blockIdx.x * QT + threadIdx.x) * 4;
    const bool in = i4 < n;  // n % 32 == 0: groups are whole
    const float4 w = in ? *(const float4*)(m + i4) : make_float4(0.f, 0.f, 0.f, 0.f);
    float amax = sw_max(sw_max(fabsf(w.x), fabsf(w.y)), sw_max(fabsf(w.z), fabsf(w.w)));
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) amax = sw_max(amax, __shfl_xor(amax, o));
    uint16_t sh = f2h(amax / 127.0f);
    if (h2f(sh) * 127.0f < amax) sh = (uint16_t)(sh + 1u);  // Convert.swift:229
    const float s = h2f(sh);
    const float inv = s > 0.0f ? 1.0f / s : 0.0f;
    if (in) {
        const float v[4] = {w.x, w.y, w.z, w.w};
        uint32_t word = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k)
            word |= (uint32_t)(uint8_t)(int8_t)sw_max(-127.0f, sw_min(127.0f, roundf(v[k] * inv))) << (8 * k);
        *(uint32_t*)(codes + i4) = word;
        if ((i4 & 31) == 0) scales[i4 >> 5] = sh;
    }
}

__device__ __forceinline__ float code_of(float w, float b, float inv) {
#pragma clang fp contract(off)
    return sw_min(15.0f, sw_max(0.0f, roundf((w - b) * inv)));
}

__global__ __launch_bounds__(QT) void quant_q4_kernel(const float* __restrict__ m, int64_t ngroups,
                                                      uint8_t* __restrict__ packed, uint16_t* __restrict__ sb,
                                                      uint8_t* __restrict__ none) {
#pragma clang fp contract(off)
    const int64_t gi = (int64_t)blockIdx.x * QT + threadIdx.x;
    if (gi >= ngroups) return;
    float w[64];
    const float4* src = (const float4*)(m + gi * 64);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const float4 v = src[k];
        w[4 * k] = v.x;
        w[4 * k + 1] = v.y;
        w[4 * k + 2] = v.z;
        w[4 * k + 3] = v.w;
    }
    float mn = w[0], mx = w[0];
#pragma unroll
    for (int i = 1; i < 64; ++i) {
        mn = sw_min(mn, w[i]);
        mx = sw_max(mx, w[i]);
    }
    uint32_t best[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint16_t best_s = 0, best_b = 0;
    bool accepted = false;
    if (mx - mn < 1e-12f) {  // constant group: codes 0, (0, mn)
        best_b = f2h(mn);
        accepted = true;
    } else {
        // The reference accumulates Σw inside every candidate's loop; the sequence is the same
        // each time, so one in-order sum gives the same value.
        float sw = 0.0f;
#pragma unroll
        for (int i = 0; i < 64; ++i) sw += w[i];
        const float clips[5] = {0.0f, 0.03f, 0.06f, 0.1f, 0.15f};
        const float range = mx - mn;
        float best_err = __builtin_inff();
        for (int ai = 0; ai < 5; ++ai) {
            for (int cj = 0; cj < 5; ++cj) {
                const float lo = mn + clips[ai] * range, hi = mx - clips[cj] * range;
                if (hi <= lo) continue;
                float s = (hi - lo) / 15.0f, b = lo;
                {
                    const float inv = 1.0f / s;
                    float sq = 0.0f, sqq = 0.0f, sqw = 0.0f;
#pragma unroll
                    for (int i = 0; i < 64; ++i) {
                        const float v = code_of(w[i], b, inv);
                        sq += v;
                        sqq += v * v;
                        sqw += v * w[i];
                    }
                    const float den = 64.0f * sqq - sq * sq;
                    if (den > 0.0f) {
                        const float s2 = (64.0f * sqw - sq * sw) / den;
                        if (s2 > 0.0f) {
                            s = s2;
                            b = (sw - s2 * sq) / 64.0f;
                        }
                    }
                }
                const uint16_t sh = f2h(s), bh = f2h(b);
                const float sf = h2f(sh), bf = h2f(bh);
                if (sf <= 0.0f) continue;
                const float inv = 1.0f / sf;
                float err = 0.0f;
                uint32_t cur[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    uint32_t word = 0;
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        const int i = 8 * j + t;
                        const float v = code_of(w[i], bf, inv);
                        word |= (uint32_t)v << (4 * t);  // q[2k] low nibble, q[2k + 1] high
                        const float d = sf * v + bf - w[i];
                        err += d * d;
                    }
                    cur[j] = word;
                }
                if (err < best_err) {
                    best_err = err;
                    best_s = sh;
                    best_b = bh;
#pragma unroll
                    for (int j = 0; j < 8; ++j) best[j] = cur[j];
                    accepted = true;
                }
            }
        }
    }
    uint4* dst = (uint4*)(packed + gi * 32);
    dst[0] = make_uint4(best[0], best[1], best[2], best[3]);
    dst[1] = make_uint4(best[4], best[5], best[6], best[7]);
    *(uint32_t*)(sb + gi * 2) = (uint32_t)best_s | ((uint32_t)best_b << 16);
    none[gi] = accepted ? 0 : 1;
}

// Groups that accepted no candidate take the codes of the nearest previous group of their
// 64-row chunk that did (or was constant); none at the chunk start: zeros.
__global__ __launch_bounds__(QT) void quant_q4_carry_kernel(int64_t ngroups, int64_t chunk_groups,
                                                            uint8_t* __restrict__ packed,
                                                            const uint8_t* __restrict__ none) {
    const int64_t gi = (int64_t)blockIdx.x * QT + threadIdx.x;
    if (gi >= ngroups || !none[gi]) return;
    const int64_t c0 = gi / chunk_groups * chunk_groups;
    uint4 lo = make_uint4(0u, 0u, 0u, 0u), hi = lo;
    for (int64_t g = gi - 1; g >= c0; --g) {
        if (!none[g]) {
            lo = ((const uint4*)(packed + g * 32))[0];
            hi = ((const uint4*)(packed + g * 32))[1];
            break;
        }
    }
    ((uint4*)(packed + gi * 32))[0] = lo;
    ((uint4*)(packed + gi * 32))[1] = hi;
}

}  // namespace

// Static scratch of the allocation-free quantiser entry point: the q4 kernel's per-group "no
// candidate accepted" byte, for up to QUANT_SCRATCH_GROUPS 64-weight groups (8 MiB, 512 M
// weights: every matrix of the decoder, the 151936 x 2048 embedding included).  Each GPU the
// library runs on holds its own copy for the life of the process.  Host code never names the
// array: it passes the device address that hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) uint8_t scratch[QUANT_SCRATCH_GROUPS];

hipError_t quant_scratch(uint8_t** out) {
    // One lookup per device, with that device current (the caller's), kept for later calls.
    static std::mutex mu;
    static uint8_t* ptrs[QUANT_MAX_DEVICES] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= QUANT_MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!ptrs[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        ptrs[dev] = (uint8_t*)p;
    }
    *out = ptrs[dev];
    return hipSuccess;
}

hipError_t launch_quant(int fmt, const float* m, int64_t rows, int64_t cols, void* codes, void* sb, uint8_t* none,
                        hipStream_t s) {
    const int64_t n = rows * cols;
    if (fmt == FMT_Q8) {
        hipLaunchKernelGGL(quant_q8_kernel, dim3((unsigned)((n / 4 + QT - 1) / QT)), dim3(QT), 0, s, m, n,
                           (int8_t*)codes, (uint16_t*)sb);
        return hipGetLastError();
    }
    if (fmt != FMT_Q4) return hipErrorInvalidValue;
    const int64_t ng = n / 64;
    const dim3 grid((unsigned)((ng + QT - 1) / QT));
    hipLaunchKernelGGL(quant_q4_kernel, grid, dim3(QT), 0, s, m, ng, (uint8_t*)codes, (uint16_t*)sb, none);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(quant_q4_carry_kernel, grid, dim3(QT), 0, s, ng, 64 * (cols / 64), (uint8_t*)codes,
                       (const uint8_t*)none);
    return hipGetLastError();
}

}  // namespace icua
