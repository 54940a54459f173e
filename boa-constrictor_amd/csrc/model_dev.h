// Per-element model arithmetic shared by every model kernel of libboa_hip.so (the tiled GEMMs, the
// LayerNorm / conv / scan kernels and the fused decompress-step kernel).  Each function below is the one
// place its expression is written: the compress path and the decompress path call the same code, which is
// what keeps their logits bit-identical (with -ffp-contract=off every operation rounds once as written).
#pragma once

#include "boa_common.h"

namespace boa {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Pointers into device global memory (address space 1).  A pointer the kernel reads from memory (a per-layer
// table, say) is generic to the compiler, which then emits FLAT loads; FLAT loads also count against the LDS
// counter, so every wait on an LDS read would also wait on them.  Casting to the global space gives global
// loads and stores.
template <class T> using gptr = __attribute__((address_space(1))) const T*;
template <class T> using gmut = __attribute__((address_space(1))) T*;
template <class T> __device__ __forceinline__ gptr<T> G(const T* p) { return (gptr<T>)p; }
template <class T> __device__ __forceinline__ gmut<T> GM(T* p) { return (gmut<T>)p; }
// 16-byte global loads and stores through native vector types (HIP's float4 / uint4 are classes, whose
// members cannot be used on an address-space-qualified object)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
template <class T> __device__ __forceinline__ u32x4 ldg16(gptr<T> p) { return *(gptr<u32x4>)p; }
template <class T> __device__ __forceinline__ float4 ldg_f4(gptr<T> p) {
    const f32x4 v = *(gptr<f32x4>)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
template <class T> __device__ __forceinline__ void stg_f4(gmut<T> p, float4 v) { *(gmut<f32x4>)p = f32x4{v.x, v.y, v.z, v.w}; }

// Raw buffer access (no swizzle, stride 0) over [base, base + nbytes): a load past the end returns 0 and a store
// past the end is dropped, so loads and stores of rows that may not exist need no branch.  The whole byte
// offset goes in the vector operand (the range check does not include the scalar offset).  Word 3 of the
// descriptor for the gfx9 family (gfx950): 32-bit data format.
// All of these accesses are non-temporal (cache policy bit NT): they are used for recurrent state that each
// step reads once and writes once, and the streaming policy keeps that traffic from evicting the GEMM weights,
// which every workgroup re-reads from L2.
constexpr int BUF_WORD3 = 0x00020000;
constexpr int CPOL_NT = 2;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nbytes, BUF_WORD3);
}
typedef uint32_t bufv4 __attribute__((vector_size(16)));
__device__ __forceinline__ f32x4 buf_ld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CPOL_NT));
}
__device__ __forceinline__ void buf_st4(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(bufv4, v), r, off, 0, CPOL_NT);
}
// 16 bytes through a buffer descriptor with the default cache policy (data that other workgroups re-read)
__device__ __forceinline__ u32x4 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float buf_ld1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CPOL_NT));
}
__device__ __forceinline__ void buf_st1(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off, 0, CPOL_NT);
}

// Fragment-packed weight blocks read through a buffer descriptor: each lane's 16 bytes sit at lane * 16 in the
// vector operand (a per-thread constant) and the block's byte offset, which is uniform, in the scalar operand, so a
// load needs no vector address arithmetic.  (With 64-bit global addresses every load costs two vector adds, which
// compete with the MFMAs for issue: an isolated fp32 decode GEMM phase measured 18.8-20 us against 15.1-15.3 us.)
// The range is not used for bounds (every block read lies inside its matrix): it is the largest one.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t wbuf(const void* base) { return buf_rsrc(base, 0xFFFFFFFFu); }
// 16 bytes of block `blk` (blocks of `blk_bytes` bytes), the lane's part at lane_off = lane * 16 bytes (plus
// part_off bytes for a second part of the block)
__device__ __forceinline__ u32x4 wbuf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t lane_off, uint32_t blk_byte_off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, lane_off, blk_byte_off, 0));
}

__device__ __forceinline__ float gelu_erf(float v);  // below

// GEMM epilogues: none | +bias | +bias,GELU(erf) | +bias,ReLU | residual + (acc + bias)
enum { EPI_NONE = 0, EPI_BIAS = 1, EPI_GELU = 2, EPI_RELU = 3, EPI_RESID = 4 };

// Quantiser precision of the fused coder (bits of the CDF total).
static constexpr int CODER_P = 24;


// Epilogue value of one accumulator before the residual add (EPI_RESID adds bias here, residual later).
template <int EPI>
__device__ __forceinline__ float epi_value(float acc, float bias) {
    float v = acc;
    if constexpr (EPI != EPI_NONE) v = v + bias;
    if constexpr (EPI == EPI_GELU) v = gelu_erf(v);
    if constexpr (EPI == EPI_RELU) v = fmaxf(v, 0.0f);
    return v;
}

// fp32 -> bfloat16, round to nearest even, two at a time (v_cvt_pk_bf16_f32; a in the low half).  Its bits
// equal the integer rounding (u + 0x7FFF + lsb) >> 16 for every finite fp32 value below 3e38 in magnitude
// (checked exhaustively over all 2^32 bit patterns on gfx950).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16_pk(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
__device__ __forceinline__ uint32_t bf16_rne(float f) { return bf16_pk(f, 0.0f) & 0xFFFFu; }

// f = hi + lo (+ a remainder below 2^-16 of f): both parts bfloat16, hi = RNE(f), lo = RNE(f - hi)
__device__ __forceinline__ void split2(float f, uint32_t& hi, uint32_t& lo) {
    hi = bf16_rne(f);
    lo = bf16_rne(f - __uint_as_float(hi << 16));
}
// The same for a pair, packed (a in the low halves): 4 instructions for both values.
__device__ __forceinline__ void split2x2(float a, float b, uint32_t& hp, uint32_t& lp) {
    hp = bf16_pk(a, b);
    lp = bf16_pk(a - __uint_as_float(hp << 16), b - __uint_as_float(hp & 0xFFFF0000u));
}
// Four consecutive values: hp / lp hold the 4 hi / lo parts in order (one 8-byte store each).
__device__ __forceinline__ void split4(float a, float b, float c, float d, uint2& hp, uint2& lp) {
    split2x2(a, b, hp.x, lp.x);
    split2x2(c, d, hp.y, lp.y);
}

// Eight consecutive fp32 values as split bf16 operands (hi, lo) of one MFMA K slice.
__device__ __forceinline__ void split8(const float* v, bf16x8& ah, bf16x8& al) {
    uint32_t hh[4], ll[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) split2x2(v[2 * e], v[2 * e + 1], hh[e], ll[e]);
    ah = __builtin_bit_cast(bf16x8, make_uint4(hh[0], hh[1], hh[2], hh[3]));
    al = __builtin_bit_cast(bf16x8, make_uint4(ll[0], ll[1], ll[2], ll[3]));
}

// LayerNorm statistics of a row of 256 * LNV values held by one wavefront, lane j holding elements
// 256 * i + 4j .. 256 * i + 4j + 3 in v[4i .. 4i + 3].  Biased variance, eps 1e-5 (nn.LayerNorm).
template <int LNV>
__device__ __forceinline__ void ln_stats_row(const float (&v)[4 * LNV], float& mu, float& rs) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4 * LNV; ++i) s = s + v[i];
    s = wave_sum(s);
    mu = s / (float)(256 * LNV);
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < 4 * LNV; ++i) {
        const float d = v[i] - mu;
        sq = sq + d * d;
    }
    sq = wave_sum(sq);
    const float var = sq / (float)(256 * LNV);
    rs = 1.0f / sqrtf(var + 1e-5f);
}

__device__ __forceinline__ float ln_apply(float v, float mu, float rs, float w, float b) { return ((v - mu) * rs) * w + b; }

// One 32-wide K step of a split-precision product into acc: a = ah + al (activations), w = bh (+ bl): the
// products lo*hi, hi*lo (NT = 3 only), hi*hi, in this order.  Every split-mode GEMM accumulates its K steps
// through this sequence.
//
// NT = 1 is the fp32 mode: the 32-wide K step is two 16-K groups of v_mfma_f32_16x16x4_f32, in the order of the
// tiled fp32 GEMM (k_gemm): group 2s, then 2s + 1, and within a group the MFMA j (j < 4) takes k = 16 g +
// 4 (l / 16) + j from lane l.  The 16-byte operands then hold fp32 values: ah = lane l's 4 values of group 2s,
// al = those of group 2s + 1 (fp32 activations are stored in the split operand's two arrays for that, see
// f32_col), and the weight block likewise (bh: group 2s, bl: group 2s + 1; two 1 KB blocks, as bf16x3's hi and lo).
__device__ __forceinline__ floatx4 mfma_f32_group(floatx4 acc, bf16x8 a, bf16x8 b) {
    const f32x4 av = __builtin_bit_cast(f32x4, a), bv = __builtin_bit_cast(f32x4, b);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[0], bv[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[1], bv[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[2], bv[2], acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x4f32(av[3], bv[3], acc, 0, 0, 0);
}
template <int NT>
__device__ __forceinline__ floatx4 mfma_split_step(floatx4 acc, bf16x8 ah, bf16x8 al, bf16x8 bh, bf16x8 bl) {
    if constexpr (NT == 1) return mfma_f32_group(mfma_f32_group(acc, ah, bh), al, bl);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
    if constexpr (NT == 3) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
}
// Fragment-packed weight blocks come in two 1 KB halves per K step in the bf16x3 (hi, lo) and fp32 (groups 2s,
// 2s + 1) modes, and as one 1 KB block in bf16w.
template <int NT> constexpr bool two_part_blocks() { return NT != 2; }
// fp32 activations in a split operand's layout (NT = 1): values k .. k + 3 of a row (k % 4 == 0) form one 16-byte
// chunk of the "hi" array for k % 32 < 16, of the "lo" array otherwise, at the bf16 column f32_col(k), so that
// the split kernels' 16-byte fragment reads (bf16 column 32 s + 8 (l / 16)) return a lane's group values.
__device__ __forceinline__ int f32_col(int k) { return 32 * (k >> 5) + 2 * (k & 15); }
__device__ __forceinline__ bool f32_lo(int k) { return (k & 16) != 0; }

// The same step with the operand roles swapped: acc^T += B^T A^T, i.e. the output fragment transposed (lane l
// holds column 4 (l / 16) + r, row l % 16).  Each output element gets the same three products (exact in fp32)
// summed over the same K slice in the same order, so it equals mfma_split_step's bit for bit.  Used where the
// fragment-packed weight block is the A operand, which makes a lane's 4 outputs consecutive columns.
template <int NT>
__device__ __forceinline__ floatx4 mfma_split_step_t(floatx4 acc, bf16x8 ah, bf16x8 al, bf16x8 bh, bf16x8 bl) {
    if constexpr (NT == 1) return mfma_f32_group(mfma_f32_group(acc, bh, ah), bl, al);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh, al, acc, 0, 0, 0);
    if constexpr (NT == 3) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bl, ah, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh, ah, acc, 0, 0, 0);
}

// Keeps the memory loads issued so far at this point of the schedule (ALU, MFMA and LDS instructions may still
// move across).  Without it the scheduler sinks a register ring's prefetches down to their uses, and the ring
// no longer hides any latency.
__device__ __forceinline__ void pin_loads() { asm volatile("" ::: "memory"); }

// x_proj (d_inner -> dt_rank + 2 d_state) is a sum of K-block partials in every precision mode:
//   dbc = P_0 + P_1 + ... + P_{d_inner/64 - 1}   (left to right, fp32 adds)
// where P_q accumulates the two 32-wide K steps (four 16-K groups in the fp32 mode) of channels 64q .. 64q + 63
// from zero.  The fused decode kernels compute P_q in the wavefront that produced those channels' conv outputs,
// so x_proj starts without a workgroup barrier; the compress and per-layer paths compute the same partials and
// the same fold.
constexpr int XPROJ_KB = 64;

// Activations on the hardware transcendental units (v_exp_f32 = 2^x, v_log_f32 = log2 x, v_rcp_f32 = 1/x,
// each within about 1 ulp).  Relative error of the results below is a few 1e-7, far inside the 1e-4
// logits tolerance against the fp32 reference, and a fraction of the instructions of expf / log1pf / IEEE
// division.  Encoder and decoder share these functions, so their logits stay bit-identical.
__device__ __forceinline__ float hw_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }
// x * sigmoid(x) = x / (1 + e^-x)
__device__ __forceinline__ float hw_silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + hw_exp(-x)); }
// softplus(x) = log(1 + e^x) (F.softplus: x itself above 20), as max(x, 0) + log1p(e^-|x|); log1p(e) for
// e in (0, 1] as log(u) * e / (u - 1) with u = 1 + e (Goldberg), exact to rounding also when u rounds to 1.
// No branch for F.softplus's threshold: above 20, e < 2^-28 rounds u to 1, so l1p = e, and x + e rounds to x
// (e is below half an ulp of x), which is the thresholded value bit for bit.
__device__ __forceinline__ float hw_softplus(float x) {
    const float e = hw_exp(-fabsf(x));
    const float u = 1.0f + e;
    const float d = u - 1.0f;
    const float l1p = (d == 0.0f) ? e : (__builtin_amdgcn_logf(u) * 0.693147180559945309f) * (e * __builtin_amdgcn_rcpf(d));
    return fmaxf(x, 0.0f) + l1p;
}

// GELU (erf form, nn.GELU()) = (x / 2) (1 + erf(x / sqrt 2)), with erf from Abramowitz & Stegun 7.1.26:
// erf(u) = 1 - q, q = t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) e^{-u^2}, t = 1 / (1 + p u), u >= 0 (absolute
// error below 1.5e-7).  (1 + erf) / 2 is formed as 1 - q / 2 or q / 2 directly, so there is no cancellation
// for negative x.  Folded for the VALU: the a_i are halved (exact), so the polynomial yields q / 2; p u =
// (p / sqrt 2) |x|; e^{-u^2} = 2^{-w^2} with w = |x| sqrt(log2(e) / 2); Horner steps are fused multiply-adds.
// 16 instructions per value.  Absolute error of the result below 4.3e-7 (checked against float64 on [-12, 12]).
__device__ __forceinline__ float gelu_erf(float v) {
    const float a = fabsf(v);
    const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.231641889f, a, 1.0f));
    float p = __builtin_fmaf(0.5307027145f, t, -0.7265760135f);
    p = __builtin_fmaf(p, t, 0.7107068705f);
    p = __builtin_fmaf(p, t, -0.142248368f);
    p = __builtin_fmaf(p, t, 0.127414796f);
    const float w = a * 0.849321800288f;
    const float qh = (p * t) * __builtin_amdgcn_exp2f(-(w * w));
    return v * (v >= 0.0f ? 1.0f - qh : qh);
}

// Depthwise causal conv (d_conv = 4) + bias + SiLU of one channel at one position:
// xc = b + w0*x[t-3] + w1*x[t-2] + w2*x[t-1] + w3*x[t] (model.py:72, PyTorch Conv1d cross-correlation).
__device__ __forceinline__ float conv_point(const float4 w, float bias, float h0, float h1, float h2, float x) {
    float v = bias;
    v = __builtin_fmaf(w.x, h0, v);
    v = __builtin_fmaf(w.y, h1, v);
    v = __builtin_fmaf(w.z, h2, v);
    v = __builtin_fmaf(w.w, x, v);
    return hw_silu(v);
}

// Selective scan, one position of one channel (Mamba's selective_scan_fn on one step):
//   dt = softplus(dr . dt_w[c] + dt_b[c])     (threshold 20 as F.softplus)
//   h_n <- exp(dt * A_n) * h_n + B_n * (dt * x) ;  with a[n] = A_n * log2(e) so exp(dt*A_n) = exp2(dt*a[n])
//   y = sum_n h_n * C_n + D * x ;  y <- y * SiLU(z)
// row = [dr (R) | B (NS) | C (NS)] of the position.
// The two halves of a position, for callers that compute dt ahead of the state update (same operations):
// scan_dt: dt of the position (uses row[0 .. R-1]); scan_update: state update, output and gate.
template <int R>
__device__ __forceinline__ float scan_dt(const float* row, const float (&wr)[R], float bdt) {
    float dt = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) dt = __builtin_fmaf(row[r], wr[r], dt);
    dt = dt + bdt;
    return hw_softplus(dt);
}
// INPLACE: the state update as one v_fma_f32 whose result overwrites h_n's own register (the same fused
// multiply-add).  In a loop over positions the compiler otherwise accumulates into dBx's register (v_fmac), so
// the new h_n lands in another register than the old and the loop rotates all NS of them with moves each
// position.  dA comes from v_exp_f32, a transcendental: the hardware needs one wait state before a VALU
// instruction reads a transcendental's result, which the compiler inserts before its own instructions but not
// before inline assembly, hence the s_nop 0 (without it the v_fma_f32 reads a stale dA).  (Pairs of updates in
// one block with the exponentials two instructions ahead, and exponentials computed 4, 8 or 16 states ahead,
// measured 2-4% slower in the compress scan at d_model 512.)
template <int NS, int R, bool INPLACE = false>
__device__ __forceinline__ float scan_update(const float* row, float dt, const float (&a)[NS], float Dc, float x, float z,
                                             float (&h)[NS]) {
    float y = 0.0f;
    const float dtx = dt * x;
#pragma unroll
    for (int n = 0; n < NS; ++n) {
        const float dA = __builtin_amdgcn_exp2f(dt * a[n]);  // v_exp_f32
        const float dBx = row[R + n] * dtx;
        if constexpr (INPLACE) __asm__("s_nop 0\n\tv_fma_f32 %0, %1, %0, %2" : "+v"(h[n]) : "v"(dA), "v"(dBx));
        else h[n] = __builtin_fmaf(dA, h[n], dBx);
        y = __builtin_fmaf(h[n], row[R + NS + n], y);
    }
    y = __builtin_fmaf(Dc, x, y);
    return y * hw_silu(z);
}
template <int NS, int R, bool INPLACE = false>
__device__ __forceinline__ float scan_position(const float* row, const float (&wr)[R], float bdt, const float (&a)[NS],
                                               float Dc, float x, float z, float (&h)[NS]) {
    return scan_update<NS, R, INPLACE>(row, scan_dt<R>(row, wr, bdt), a, Dc, x, z, h);
}

// Logits of one lane (a V-wide row) as held by one wavefront: lane j gets elements 4j .. 4j + 3 (0 beyond V).
__device__ __forceinline__ float4 logits_row4(const float* row, int V, int lane) {
    float4 l4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (4 * lane + 3 < V) {
        l4 = *reinterpret_cast<const float4*>(row + 4 * lane);
    } else {
        if (4 * lane + 0 < V) l4.x = row[4 * lane + 0];
        if (4 * lane + 1 < V) l4.y = row[4 * lane + 1];
        if (4 * lane + 2 < V) l4.z = row[4 * lane + 2];
    }
    return l4;
}

// Chunk b's stream inside a payload of `total` words: words [off[b], off[b] + nwords[b]) clamped to
// [0, total).  Offsets or counts that do not fit the payload then read zeros, as the decoder reads zeros
// past the end of any stream, and no word outside the payload is read (the file reader's bound,
// boa.cpp:240, enforced on the device for callers that pass arbitrary offsets).
struct LaneWords {
    const uint32_t* p;
    int32_t n;
};
__device__ __forceinline__ LaneWords lane_words(const uint32_t* payload, int64_t total, const int64_t* off,
                                                const int32_t* nwords, int64_t b) {
    int64_t o = off[b];
    o = o < 0 ? 0 : (o > total ? total : o);
    int64_t n = nwords[b];
    n = n < 0 ? 0 : (n > total - o ? total - o : n);
    return {payload + o, (int32_t)n};
}

// One decode step of one lane (whole wavefront): quantise the logits (XQ), find the symbol the coder state
// points into, advance the state.  Returns the symbol (uniform across the wave).
__device__ __forceinline__ int decode_row(const float* row, int V, int lane, DecState& st, const uint32_t* in,
                                          int32_t nw) {
    XQ q;
    xq_build(q, logits_row4(row, V, lane), lane, V, CODER_P);
    uint32_t e[4];
    uint32_t c = q.base;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = 4 * lane + j;
        e[j] = (k < V) ? xq_cdf_at(q, c, k) : (1u << CODER_P);
        c += q.f[j];
    }
    const uint32_t qv = dec_target(st, CODER_P);
    uint32_t lo, hi;
    const int s = wave_find_symbol<CODER_P>(e, V, qv, lane, lo, hi);
    dec_advance(st, CODER_P, lo, hi - lo, in, nw);
    return s;
}

}  // namespace boa
