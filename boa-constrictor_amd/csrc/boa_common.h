// Device-side building blocks shared by every kernel of libboa_hip.so (gfx950, wave64).
//
// Compiled with -ffp-contract=off: every floating-point expression below rounds once per operation, as
// written, so that (a) the compress path (many positions per launch) and the decompress path (one
// position per launch) execute identical arithmetic per element and produce identical logits, and (b) the
// fused quantiser can be restated bit-exactly on the CPU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define BOA_WAVE 64
#define BOA_HD __host__ __device__ __forceinline__
#include "rc_core.h"

namespace boa {

// ------------------------------------------------------------------------------------------------
// exp used by the fused quantiser: Cody & Waite (1980) reduction x = k*ln2 + r with ln2 split into a
// 16-significant-bit head (k*LN2_HI exact for |k| < 256) and a tail, the degree-7 Taylor polynomial of
// e^r in Horner form, and scaling by 2^k (v_ldexp_f32).  Max error about 2 ulp.  Inputs below -87 (and
// NaN) give 0, which the quantiser's 2^23 fixed-point step maps to 0 anyway.
__device__ __forceinline__ float boa_expf(float x) {
    if (!(x >= -87.0f)) return 0.0f;
    if (x > 88.0f) x = 88.0f;
    const float kf = __builtin_rintf(x * 0x1.715476p+0f);
    float r = x - kf * 0x1.62e4p-1f;
    r = r - kf * 0x1.7f7d1cp-20f;
    float p = 0x1.a01a02p-13f;
    p = p * r + 0x1.6c16c2p-10f;
    p = p * r + 0x1.111112p-7f;
    p = p * r + 0x1.555556p-5f;
    p = p * r + 0x1.555556p-3f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return __builtin_ldexpf(p, (int)kf);
}

// ------------------------------------------------------------------------------------------------
// Wavefront collectives.  Butterfly (xor) reductions leave the same value in every lane; all orders are
// fixed by the lane index only, never by timing.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, BOA_WAVE));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o, BOA_WAVE);
    return v;
}

// Inclusive prefix sum of unsigned 32-bit values across the wave (exact: integer adds).
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v, int lane) {
#pragma unroll
    for (int o = 1; o < BOA_WAVE; o <<= 1) {
        uint32_t t = __shfl_up(v, o, BOA_WAVE);
        if (lane >= o) v += t;
    }
    return v;
}

template <typename T>
__device__ __forceinline__ T wave_bcast(T v, int src) { return __shfl(v, src, BOA_WAVE); }

// ------------------------------------------------------------------------------------------------
// Range-coder core (EncState/DecState, enc_push, enc_finish, dec_init, dec_target, dec_advance): rc_core.h,
// shared with the host build that checks it on the CPU.

// ------------------------------------------------------------------------------------------------
// Fused quantiser (XQ), wave-parallel: lane j owns symbols 4j..4j+3 (vocab <= 256).
//   m = max l;  e = boa_expf(l - m);  f = trunc(e * 2^23);  c_i = sum_{j<i} f_j (exact integers)
//   cdf_i = (u32)((double)c_i * ((double)(2^P - V) / (double)S)) + i,  cdf_V = 2^P
// The CPU restatement is ora_xq_cdf in oracle/rc_oracle.c.
struct XQ {
    uint32_t f[4];     // fixed-point weights of this lane's symbols
    uint32_t base;     // c of this lane's first symbol
    uint32_t S;        // total
    double inv;        // (2^P - V) / S
    bool uniform;      // S == 0 fallback (uniform table, as Q2's degenerate branch)
    uint32_t ustep;    // (2^P - V) / V + 1 for the uniform fallback
};

__device__ __forceinline__ void xq_build(XQ& q, const float4 l4, int lane, int V, int P) {
    const int k0 = 4 * lane;
    float l[4] = {l4.x, l4.y, l4.z, l4.w};
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int j = 0; j < 4; ++j) if (k0 + j < V) mx = fmaxf(mx, l[j]);
    mx = wave_max(mx);
    uint32_t loc = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t f = 0u;
        if (k0 + j < V) f = (uint32_t)(boa_expf(l[j] - mx) * 8388608.0f);
        q.f[j] = f;
        loc += f;
    }
    const uint32_t incl = wave_incl_scan_u32(loc, lane);
    q.base = incl - loc;
    q.S = wave_bcast(incl, BOA_WAVE - 1);
    const uint32_t free_w = (1u << P) - (uint32_t)V;
    q.uniform = (q.S == 0u);
    q.ustep = free_w / (uint32_t)V + 1u;
    q.inv = q.uniform ? 0.0 : (double)free_w / (double)q.S;
}

// cdf value of symbol i given its exact cumulative c (i < V)
__device__ __forceinline__ uint32_t xq_cdf_at(const XQ& q, uint32_t c, int i) {
    if (q.uniform) return (uint32_t)i * q.ustep;
    return (uint32_t)((double)c * q.inv) + (uint32_t)i;
}

// Loads this lane's 4 table entries of one row (entries >= K read as 2^P, i.e. never <= target).
template <int P, typename TC>
__device__ __forceinline__ void load_row4(const TC* row, int K, int lane, uint32_t e[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = 4 * lane + j;
        e[j] = (k < K) ? (uint32_t)row[k] : (1u << P);
    }
}

// Symbol lookup with the reference decoder's semantics (gpu_range_coder.py:196-198): the smallest
// i in [1, K] with cdf[i] > q (cdf[K] = 2^P), minus one, clamped to [0, K-1].  Entries are held 4 per
// lane (lane j: 4j..4j+3).  Returns s and the entries cdf[s], cdf[s+1].
template <int P>
__device__ __forceinline__ int wave_find_symbol(const uint32_t e[4], int K, uint32_t q, int lane,
                                                uint32_t& lo, uint32_t& hi) {
    int best = K;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = 4 * lane + j;
        const bool pred = (k >= 1) && (k < K) && (e[j] > q);
        const uint64_t m = __ballot(pred);
        if (m) {
            const int first_lane = __builtin_ctzll(m);
            const int idx = 4 * first_lane + j;
            best = idx < best ? idx : best;
        }
    }
    int s = best - 1;
    if (s < 0) s = 0;
    if (s >= K) s = K - 1;
    // fetch cdf[s] and cdf[s+1] from their owner lanes (s uniform across the wave)
    const int js = s & 3, jn = (s + 1) & 3;
    const uint32_t vs = js == 0 ? e[0] : js == 1 ? e[1] : js == 2 ? e[2] : e[3];
    const uint32_t vn = jn == 0 ? e[0] : jn == 1 ? e[1] : jn == 2 ? e[2] : e[3];
    lo = wave_bcast(vs, s >> 2);
    hi = (s + 1 < K) ? wave_bcast(vn, (s + 1) >> 2) : (1u << P);
    return s;
}

}  // namespace boa

// Error-checked launch helper for host code.
#define BOA_HIP_TRY(expr)                                                                           \
    do {                                                                                            \
        hipError_t _e = (expr);                                                                     \
        if (_e != hipSuccess) return boa_fail_hip(_e, #expr, __FILE__, __LINE__);                   \
    } while (0)

int boa_fail(int code, const char* fmt, ...);
int boa_fail_hip(hipError_t e, const char* what, const char* file, int line);
