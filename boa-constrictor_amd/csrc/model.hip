// Model kernels and the model context of libboa_hip.so: BoaBytePredictor (embedding, L blocks of
// LayerNorm -> Mamba mixer -> LayerNorm -> GELU feed-forward with a block residual, Linear-ReLU-Linear head)
// for many chunk lanes at once, plus the fused compress / decompress drivers.
//
// Row layout: a launch processes B lanes x Tc positions; row m = b * Tc + t.  The same kernels serve the
// compress path (Tc = tile length, model parallel in time) and the decompress path (Tc = 1, one recurrent
// step).  Per-element arithmetic never depends on Tc or on a row's position in a tile:
//   - GEMMs accumulate each output over K in a fixed order (16-wide K groups, 4 MFMA steps each), with
//     no split-K, so the result of a row does not depend on M or on the tile it falls in;
//   - LayerNorm statistics are wave reductions over the row only;
//   - the conv and selective-scan kernels run the same per-position code whether the state comes from
//     registers (previous position in the same tile) or from HBM (previous launch).
// This is what makes the encoder's and decoder's logits bit-identical.
#include "model_dev.h"
#include "model_internal.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <algorithm>
#include <type_traits>
#include <string>
#include <vector>

#include "../../include/boa_hip.h"

using namespace boa;

// ================================================================================================
// Errors (thread-local last message)
static thread_local std::string g_last_error;

int boa_fail(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int boa_fail_hip(hipError_t e, const char* what, const char* file, int line) {
    return boa_fail(BOA_ERR_HIP, "HIP error %d (%s) in %s at %s:%d", (int)e, hipGetErrorString(e), what, file, line);
}

extern "C" const char* boa_last_error(void) { return g_last_error.c_str(); }
extern "C" int boa_abi_version(void) { return 2; }  // 2: boa_decompress takes payload_words

extern "C" int boa_is_device_pointer(const void* p) {
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return a.type == hipMemoryTypeDevice ? 1 : 0;
}

// ================================================================================================
// GEMM: C[M,N] = epilogue( prologue(A)[M,K] * W[N,K]^T )  on MFMA v_mfma_f32_16x16x4_f32.
//   A row-major (lda), W row-major [N][K] (PyTorch Linear layout, K contiguous), C row-major (ldc).
//   prologue: optional LayerNorm of each A row (K == LN width; eps 1e-5, biased variance).
//   epilogue: none | +bias | +bias,GELU(erf) | +bias,ReLU | residual + (acc + bias).
// Tiling: BM x BN per 256-thread workgroup (2 x 2 waves), BK = 32 per LDS stage, double buffered.
// Within a 16-wide K group, lane group g = lane/16 supplies k = 4g + s to MFMA step s, so each lane reads
// one float4 per fragment from LDS.  Rows of the LDS tiles are padded to 36 floats (conflict-free b128
// reads for the 16 rows a quarter-wave touches).
struct GemmArgs {
    const float* A;
    int64_t lda;
    const float* W;
    const uint16_t* Wh;  // bf16 bits of W (split precision modes)
    const uint16_t* Wl;  // bf16 bits of W - Wh (bf16x3 mode only)
    const float* bias;
    const float* R;
    int64_t ldr;
    float* C;
    int64_t ldc;
    const float* ln_w;
    const float* ln_b;
    const float2* ln_stats;  // per-row (mean, rstd) from k_ln_stats
    const uint16_t* Ah;      // pre-split A (bf16 hi / lo parts, row stride lda) instead of fp32 A
    const uint16_t* Al;
    uint16_t* Ch;            // split output (bf16 hi / lo parts, row stride ldc) instead of fp32 C
    uint16_t* Cl;
    int64_t M;
    int N;
    int K;
    int mtiles;
    int ntiles;
    int per_xcd;
};

template <int BM, int BN, int LNV, int EPI>
__global__ void __launch_bounds__(256, 2) k_gemm(GemmArgs g) {
    constexpr int BK = 32, LDK = BK + 4;
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 16, FN = WN / 16;
    constexpr int A_LD = BM * BK / 4 / 256;
    constexpr int B_LD = BN * BK / 4 / 256;
    __shared__ __attribute__((aligned(16))) float sA[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) float sB[2][BN * LDK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // XCD-aware tile order: workgroup i runs on XCD i % 8; give each XCD a contiguous range of tiles,
    // N-tiles fastest, so concurrently resident workgroups of one XCD share A rows and W in its L2.
    const int bid = blockIdx.x;
    const int tile = (bid & 7) * g.per_xcd + (bid >> 3);
    if (tile >= g.mtiles * g.ntiles) return;
    const int mt = tile / g.ntiles;
    const int nt = tile - mt * g.ntiles;
    const int64_t m0 = (int64_t)mt * BM;
    const int n0 = nt * BN;
    const int64_t M = g.M;
    const int N = g.N, K = g.K;

    float4 ra[A_LD], rb[B_LD];
    auto load_tiles = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_LD; ++i) {
            const int q = tid + 256 * i;
            const int r = q >> 3, c = (q & 7) * 4;
            const int64_t m = m0 + r;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m < M) {
                v = *reinterpret_cast<const float4*>(g.A + m * g.lda + k0 + c);
                if constexpr (LNV > 0) {
                    const float2 st = g.ln_stats[m];
                    const float mu = st.x, rs = st.y;
                    const float4 w = *reinterpret_cast<const float4*>(g.ln_w + k0 + c);
                    const float4 b = *reinterpret_cast<const float4*>(g.ln_b + k0 + c);
                    v.x = ln_apply(v.x, mu, rs, w.x, b.x);
                    v.y = ln_apply(v.y, mu, rs, w.y, b.y);
                    v.z = ln_apply(v.z, mu, rs, w.z, b.z);
                    v.w = ln_apply(v.w, mu, rs, w.w, b.w);
                }
            }
            ra[i] = v;
        }
#pragma unroll
        for (int i = 0; i < B_LD; ++i) {
            const int q = tid + 256 * i;
            const int r = q >> 3, c = (q & 7) * 4;
            const int n = n0 + r;
            rb[i] = (n < N) ? *reinterpret_cast<const float4*>(g.W + (int64_t)n * K + k0 + c)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto store_tiles = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_LD; ++i) {
            const int q = tid + 256 * i;
            *reinterpret_cast<float4*>(&sA[buf][(q >> 3) * LDK + (q & 7) * 4]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_LD; ++i) {
            const int q = tid + 256 * i;
            *reinterpret_cast<float4*>(&sB[buf][(q >> 3) * LDK + (q & 7) * 4]) = rb[i];
        }
    };

    floatx4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int KT = K / BK;
    load_tiles(0);
    store_tiles(0);
    __syncthreads();
    const int arow = wm * WM + (lane & 15);
    const int brow = wn * WN + (lane & 15);
    const int kq = 4 * (lane >> 4);
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) load_tiles((kt + 1) * BK);
#pragma unroll
        for (int kg = 0; kg < 2; ++kg) {
            float4 a[FM], b[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                a[i] = *reinterpret_cast<const float4*>(&sA[cur][(arow + 16 * i) * LDK + 16 * kg + kq]);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                b[j] = *reinterpret_cast<const float4*>(&sB[cur][(brow + 16 * j) * LDK + 16 * kg + kq]);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].x, b[j].x, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].y, b[j].y, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].z, b[j].z, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].w, b[j].w, acc[i][j], 0, 0, 0);
                }
        }
        if (kt + 1 < KT) store_tiles(cur ^ 1);
        __syncthreads();
    }

    // epilogue: lane holds rows 4*(lane/16)+r, column lane%16 of each 16x16 output fragment
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int col = n0 + wn * WN + 16 * j + (lane & 15);
            if (col >= N) continue;
            float bias = 0.0f;
            if constexpr (EPI != EPI_NONE) bias = g.bias[col];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = m0 + wm * WM + 16 * i + 4 * (lane >> 4) + r;
                if (row >= M) continue;
                float v = epi_value<EPI>(acc[i][j][r], bias);
                if constexpr (EPI == EPI_RESID) v = g.R[row * g.ldr + col] + v;
                g.C[row * g.ldc + col] = v;
            }
        }
}

// ------------------------------------------------------------------------------------------------
// Split-precision GEMM on v_mfma_f32_16x16x32_bf16.  Each fp32 activation a is split while it is staged
// into LDS as a = a_hi + a_lo (both bfloat16, round to nearest even; a - a_hi is exact in fp32), each
// weight likewise once at context creation (w = w_hi + w_lo).  With NT = 3 the product is
// a_lo*w_hi + a_hi*w_lo + a_hi*w_hi accumulated in fp32 (the a_lo*w_lo term, below 2^-16 of the product,
// is dropped); with NT = 2 the weights are bfloat16 themselves (w_lo = 0).  Products of bfloat16 pairs are
// exact in fp32, so the only losses are the dropped term and fp32 accumulation.  K order per output is
// fixed (32 per MFMA step, steps ascending), independent of M: the encoder/decoder identity holds as in
// the fp32 kernel.  LDS rows hold 32 bf16 + 8 pad (80 B: conflict-free b128 fragment reads).
// BK (K per LDS stage, a multiple of 32) changes only data movement: every output still accumulates
// 32-wide MFMA K steps in ascending order, so results do not depend on BK, BM or BN.
template <int BM, int BN, int BK, int EPI, int NT, bool ASPLIT, bool OUTS>
__global__ void __launch_bounds__(256, (BK > 32) ? 1 : 2) k_gemm_bf(GemmArgs g) {
    // LDS rows: BK = 32 tiles are unpadded (64 B per part-row) with the 16-byte chunk c of row r stored at
    // chunk c ^ ((r >> 1) & 3).  A 16-byte fragment read is served 8 lanes (128 B) at a time: 8 rows of one
    // chunk, which this puts in 8 different 16-byte bank groups (c ^ ((r >> 2) & 3) put row pairs together and
    // measured bank conflicts on 92% of LDS cycles; this, none).  Stores (rows x 4 chunks) are a permutation
    // within each row.  BK = 128 rows are padded by 8 (272 B).
    constexpr bool SWZ = (BK == 32);
    constexpr int LDK = SWZ ? BK : BK + 8;
    auto lds_off = [](int r, int k) {  // element (row r, column k) of an operand tile, k % 8 == 0 or a half chunk
        if constexpr (SWZ) return r * 32 + ((((k >> 3) ^ (r >> 1)) & 3) << 3) + (k & 7);
        else return r * LDK + k;
    };
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 16, FN = WN / 16;
    constexpr int A_LD = ASPLIT ? BM * BK / 8 / 256 : BM * BK / 4 / 256;  // per thread: 8-bf16 or float4 loads
    constexpr int B_LD = BN * BK / 8 / 256;
    // one LDS block: double-buffered bf16 operand tiles, reused for the fp32 output tile after the K loop
    constexpr int LDC = BN + 4;
    constexpr int OPER = 2 * (2 * BM * LDK + (NT == 3 ? 2 : 1) * BN * LDK);  // uint16 elements
    constexpr int OUTT = 2 * BM * LDC;                                      // uint16 elements (fp32 tile)
    __shared__ __attribute__((aligned(16))) uint16_t smem[OPER > OUTT ? OPER : OUTT];
    uint16_t (*sAh)[BM * LDK] = reinterpret_cast<uint16_t (*)[BM * LDK]>(smem);
    uint16_t (*sAl)[BM * LDK] = reinterpret_cast<uint16_t (*)[BM * LDK]>(smem + 2 * BM * LDK);
    uint16_t (*sBh)[BN * LDK] = reinterpret_cast<uint16_t (*)[BN * LDK]>(smem + 4 * BM * LDK);
    uint16_t (*sBl)[BN * LDK] = reinterpret_cast<uint16_t (*)[BN * LDK]>(smem + 4 * BM * LDK + 2 * BN * LDK);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int bid = blockIdx.x;
    const int tile = (bid & 7) * g.per_xcd + (bid >> 3);
    if (tile >= g.mtiles * g.ntiles) return;
    const int mt = tile / g.ntiles;
    const int nt = tile - mt * g.ntiles;
    const int64_t m0 = (int64_t)mt * BM;
    const int n0 = nt * BN;
    const int64_t M = g.M;
    const int N = g.N, K = g.K;

    // Operand tiles through range-checked buffer descriptors over this tile's rows of A and of W: rows past M
    // (or N) read 0 with no branch around the load, so the compiler's wait counts see every load as issued.
    const int rows_a = (int)((M - m0) < BM ? (M - m0) : BM);
    const int rows_b = (N - n0) < BN ? (N - n0) : BN;
    const __amdgpu_buffer_rsrc_t rA =
        ASPLIT ? buf_rsrc(g.Ah + m0 * g.lda, (uint32_t)(rows_a * g.lda * 2)) : buf_rsrc(g.A + m0 * g.lda, (uint32_t)(rows_a * g.lda * 4));
    const __amdgpu_buffer_rsrc_t rAl = ASPLIT ? buf_rsrc(g.Al + m0 * g.lda, (uint32_t)(rows_a * g.lda * 2)) : rA;
    const __amdgpu_buffer_rsrc_t rBh = buf_rsrc(g.Wh + (int64_t)n0 * K, (uint32_t)(rows_b * K * 2));
    const __amdgpu_buffer_rsrc_t rBl = (NT == 3) ? buf_rsrc(g.Wl + (int64_t)n0 * K, (uint32_t)(rows_b * K * 2)) : rBh;

    // Two register stages: the loads of K step kt + 2 are issued while step kt multiplies from LDS and step
    // kt + 1 (loaded during step kt - 1) is stored to the other LDS buffer, so each load has about two K
    // steps of MFMA work to arrive in.  Stage indices are compile-time (the K loop is unrolled by two).
    // A: pre-split (8 bf16 of each part per load) or fp32 split on store (4 values per load).
    u32x4 sa_h[2][A_LD], sa_l[2][ASPLIT ? A_LD : 1];
    u32x4 sb_h[2][B_LD], sb_l[2][NT == 3 ? B_LD : 1];
    auto load_tiles = [&](auto stage, int k0) {
        constexpr int S = decltype(stage)::value;
#pragma unroll
        for (int i = 0; i < A_LD; ++i) {
            const int q = tid + 256 * i;
            if constexpr (ASPLIT) {
                const int r = q / (BK / 8), c = (q % (BK / 8)) * 8;
                const uint32_t off = (uint32_t)((r * g.lda + k0 + c) * 2);
                sa_h[S][i] = buf_ld16(rA, off);
                sa_l[S][i] = buf_ld16(rAl, off);
            } else {
                const int r = q / (BK / 4), c = (q % (BK / 4)) * 4;
                sa_h[S][i] = buf_ld16(rA, (uint32_t)((r * g.lda + k0 + c) * 4));
            }
        }
#pragma unroll
        for (int i = 0; i < B_LD; ++i) {
            const int q = tid + 256 * i;
            const int r = q / (BK / 8), c = (q % (BK / 8)) * 8;
            const uint32_t off = (uint32_t)((r * K + k0 + c) * 2);
            sb_h[S][i] = buf_ld16(rBh, off);
            if constexpr (NT == 3) sb_l[S][i] = buf_ld16(rBl, off);
        }
    };
    auto store_tiles = [&](auto stage, int buf) {
        constexpr int S = decltype(stage)::value;
#pragma unroll
        for (int i = 0; i < A_LD; ++i) {
            const int q = tid + 256 * i;
            if constexpr (ASPLIT) {
                const int off = lds_off(q / (BK / 8), (q % (BK / 8)) * 8);
                *reinterpret_cast<u32x4*>(&sAh[buf][off]) = sa_h[S][i];
                *reinterpret_cast<u32x4*>(&sAl[buf][off]) = sa_l[S][i];
            } else {
                const int off = lds_off(q / (BK / 4), (q % (BK / 4)) * 4);
                const u32x4 v = sa_h[S][i];
                uint2 hp, lp;
                split4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w), hp, lp);
                *reinterpret_cast<uint2*>(&sAh[buf][off]) = hp;
                *reinterpret_cast<uint2*>(&sAl[buf][off]) = lp;
            }
        }
#pragma unroll
        for (int i = 0; i < B_LD; ++i) {
            const int q = tid + 256 * i;
            const int off = lds_off(q / (BK / 8), (q % (BK / 8)) * 8);
            *reinterpret_cast<u32x4*>(&sBh[buf][off]) = sb_h[S][i];
            if constexpr (NT == 3) *reinterpret_cast<u32x4*>(&sBl[buf][off]) = sb_l[S][i];
        }
    };

    floatx4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int KT = K / BK;
    const int arow = wm * WM + (lane & 15);
    const int brow = wn * WN + (lane & 15);
    const int kq = 8 * (lane >> 4);
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    auto multiply = [&](int cur) {
#pragma unroll
        for (int ks = 0; ks < BK; ks += 32) {
            bf16x8 ah[FM], al[FM], bh[FN], bl[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                ah[i] = *reinterpret_cast<const bf16x8*>(&sAh[cur][lds_off(arow + 16 * i, ks + kq)]);
                al[i] = *reinterpret_cast<const bf16x8*>(&sAl[cur][lds_off(arow + 16 * i, ks + kq)]);
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                bh[j] = *reinterpret_cast<const bf16x8*>(&sBh[cur][lds_off(brow + 16 * j, ks + kq)]);
                bl[j] = bh[j];
                if constexpr (NT == 3)
                    bl[j] = *reinterpret_cast<const bf16x8*>(&sBl[cur][lds_off(brow + 16 * j, ks + kq)]);
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = mfma_split_step<NT>(acc[i][j], ah[i], al[i], bh[j], bl[j]);
        }
    };
    // One K step kt with compile-time stage parity P = kt & 1: LDS buffer P holds step kt, register stage 1 - P
    // holds step kt + 1 in flight, register stage P is free.  LOAD / STORE are compile-time too: the last two
    // steps are peeled off the loop, so no load is under a branch (the compiler's wait counts would otherwise
    // make every store wait for all loads in flight).  KT is even (checked at launch).
    auto kstep = [&](auto parity, auto load, auto store, int kt) {
        constexpr int P = decltype(parity)::value;
        using SP = std::integral_constant<int, P>;
        using SQ = std::integral_constant<int, 1 - P>;
        if constexpr (decltype(load)::value) load_tiles(SP{}, (kt + 2) * BK);
        // keep the loads ahead of this step's MFMAs and the stores after them (the scheduler would sink the
        // loads below the stores, leaving them one step instead of two to arrive)
        __builtin_amdgcn_sched_barrier(0);
        multiply(P);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (decltype(store)::value) store_tiles(SQ{}, 1 - P);
        __syncthreads();
    };
    using T = std::true_type;
    using F = std::false_type;
    load_tiles(S0{}, 0);
    load_tiles(S1{}, BK);
    store_tiles(S0{}, 0);
    __syncthreads();
    for (int kt = 0; kt + 2 < KT; kt += 2) {
        kstep(S0{}, T{}, T{}, kt);
        kstep(S1{}, T{}, T{}, kt + 1);
    }
    kstep(S0{}, F{}, T{}, KT - 2);
    kstep(S1{}, F{}, F{}, KT - 1);

    // Epilogue through LDS (the operand buffers are free after the last barrier): fragments are written
    // to an fp32 tile [BM][BN + 4] (bias and activation applied here), then rows leave in 16-byte pieces.
    float* sC = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int cl = wn * WN + 16 * j + (lane & 15);
            const int col = n0 + cl;
            float bias = 0.0f;
            if constexpr (EPI != EPI_NONE) bias = (col < N) ? g.bias[col] : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                sC[(wm * WM + 16 * i + 4 * (lane >> 4) + r) * LDC + cl] = epi_value<EPI>(acc[i][j][r], bias);
        }
    __syncthreads();
    constexpr int Q = BN / 4;  // float4 pieces per tile row
#pragma unroll 4
    for (int p = tid; p < BM * Q; p += 256) {
        const int rl = p / Q, c4 = (p - rl * Q) * 4;
        const int64_t row = m0 + rl;
        const int col = n0 + c4;
        if (row >= M || col >= N) continue;  // N is a multiple of 4: a piece is all in or all out
        float4 v = *reinterpret_cast<const float4*>(&sC[rl * LDC + c4]);
        if constexpr (EPI == EPI_RESID) {
            const float4 rv = *reinterpret_cast<const float4*>(g.R + row * g.ldr + col);
            v = make_float4(rv.x + v.x, rv.y + v.y, rv.z + v.z, rv.w + v.w);
        }
        if constexpr (OUTS) {
            uint2 hp, lp;
            split4(v.x, v.y, v.z, v.w, hp, lp);
            *reinterpret_cast<uint2*>(g.Ch + row * g.ldc + col) = hp;
            *reinterpret_cast<uint2*>(g.Cl + row * g.ldc + col) = lp;
        } else {
            *reinterpret_cast<float4*>(g.C + row * g.ldc + col) = v;
        }
    }
}

static void tile_grid(GemmArgs& g, int BM, int BN, int64_t& grid) {
    g.mtiles = (int)((g.M + BM - 1) / BM);
    g.ntiles = (g.N + BN - 1) / BN;
    const int64_t tiles = (int64_t)g.mtiles * g.ntiles;
    g.per_xcd = (int)((tiles + 7) / 8);
    grid = (int64_t)g.per_xcd * 8;
}

// 128x128 when that still gives >= 2 workgroups per CU, else 64x64.
static bool big_tiles(const GemmArgs& g) {
    const int64_t big = ((g.M + 127) / 128) * (int64_t)((g.N + 127) / 128);
    return g.N >= 128 && big >= 512;
}

template <int BM, int BN, int LNV, int EPI>
static int launch_gemm_f32_cfg(GemmArgs g, hipStream_t s) {
    int64_t grid;
    tile_grid(g, BM, BN, grid);
    hipLaunchKernelGGL((k_gemm<BM, BN, LNV, EPI>), dim3((unsigned)grid), dim3(256), 0, s, g);
    return BOA_OK;
}

template <int LNV, int EPI>
static int launch_gemm_f32(const GemmArgs& g, hipStream_t s) {
    if (big_tiles(g)) return launch_gemm_f32_cfg<128, 128, LNV, EPI>(g, s);
    return launch_gemm_f32_cfg<64, 64, LNV, EPI>(g, s);
}

template <int BM, int BN, int BK, int EPI, bool ASPLIT, bool OUTS>
static int launch_gemm_bf_cfg(GemmArgs g, hipStream_t s) {
    if (g.K % (2 * BK) != 0) return boa_fail(BOA_ERR_ARG, "internal: K=%d not a multiple of 2 BK=%d", g.K, 2 * BK);
    int64_t grid;
    tile_grid(g, BM, BN, grid);
    if (g.Wl)
        hipLaunchKernelGGL((k_gemm_bf<BM, BN, BK, EPI, 3, ASPLIT, OUTS>), dim3((unsigned)grid), dim3(256), 0, s, g);
    else
        hipLaunchKernelGGL((k_gemm_bf<BM, BN, BK, EPI, 2, ASPLIT, OUTS>), dim3((unsigned)grid), dim3(256), 0, s, g);
    return BOA_OK;
}

// Shape-dependent data movement (results are independent of it, see k_gemm_bf), from a sweep on MI355X:
//   many tiles (compress, M = lanes x 64):   128x128, BK 32, 2 workgroups per CU
//   M = 4096, N >= 512 (in_proj, FF1):        64x64,  BK 32
//   M = 4096, N <= 256 (out_proj, FF2, head): 64x64,  BK 128 (fewer K stages: latency-bound shapes)
template <int EPI, bool ASPLIT, bool OUTS>
static int launch_gemm_bf(const GemmArgs& g, hipStream_t s) {
    const int64_t t128 = ((g.M + 127) / 128) * (int64_t)((g.N + 127) / 128);
    if (g.N >= 128 && t128 >= 512) return launch_gemm_bf_cfg<128, 128, 32, EPI, ASPLIT, OUTS>(g, s);
    if (g.N >= 512 || g.K % 128 != 0) return launch_gemm_bf_cfg<64, 64, 32, EPI, ASPLIT, OUTS>(g, s);
    return launch_gemm_bf_cfg<64, 64, 128, EPI, ASPLIT, OUTS>(g, s);
}

// ================================================================================================
// LayerNorm row statistics (model.py:45,51: nn.LayerNorm, eps 1e-5, biased variance): one wavefront per
// row, lane j holding elements 4j.. of each 256-wide slab; sum and sum of squared deviations by butterfly
// reduction (fixed order, identical in every lane).  The consuming GEMM applies ((x - mean) * rstd) * w + b
// while staging A.
template <int LNV>
__global__ void __launch_bounds__(256) k_ln_stats(const float* __restrict__ A, int64_t lda, int64_t M,
                                                 float2* __restrict__ stats) {
    const int lane = threadIdx.x & 63;
    const int64_t m = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (m >= M) return;
    const float* row = A + m * lda;
    float v[4 * LNV];
#pragma unroll
    for (int i = 0; i < LNV; ++i) {
        const float4 q = *reinterpret_cast<const float4*>(row + 256 * i + 4 * lane);
        v[4 * i + 0] = q.x; v[4 * i + 1] = q.y; v[4 * i + 2] = q.z; v[4 * i + 3] = q.w;
    }
    float mu, rs;
    ln_stats_row<LNV>(v, mu, rs);
    if (lane == 0) stats[m] = make_float2(mu, rs);
}

// LayerNorm of a row, written as split bfloat16 parts (hi, lo) for the split-precision GEMMs: the same
// statistics and the same ((x - mean) * rstd) * w + b expression as the fp32 path applies on load.
template <int LNV>
__global__ void __launch_bounds__(256) k_ln_split(const float* __restrict__ A, int64_t lda, int64_t M,
                                                 const float* __restrict__ w, const float* __restrict__ bvec,
                                                 uint16_t* __restrict__ Ah, uint16_t* __restrict__ Al) {
    const int lane = threadIdx.x & 63;
    const int64_t m = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (m >= M) return;
    const float* row = A + m * lda;
    float v[4 * LNV];
#pragma unroll
    for (int i = 0; i < LNV; ++i) {
        const float4 q = *reinterpret_cast<const float4*>(row + 256 * i + 4 * lane);
        v[4 * i + 0] = q.x; v[4 * i + 1] = q.y; v[4 * i + 2] = q.z; v[4 * i + 3] = q.w;
    }
    float mu, rs;
    ln_stats_row<LNV>(v, mu, rs);
#pragma unroll
    for (int i = 0; i < LNV; ++i) {
        const int c = 256 * i + 4 * lane;
        const float4 wv = *reinterpret_cast<const float4*>(w + c);
        const float4 bv = *reinterpret_cast<const float4*>(bvec + c);
        const float y[4] = {ln_apply(v[4 * i + 0], mu, rs, wv.x, bv.x), ln_apply(v[4 * i + 1], mu, rs, wv.y, bv.y),
                            ln_apply(v[4 * i + 2], mu, rs, wv.z, bv.z), ln_apply(v[4 * i + 3], mu, rs, wv.w, bv.w)};
        uint2 hp, lp;
        split4(y[0], y[1], y[2], y[3], hp, lp);
        *reinterpret_cast<uint2*>(Ah + m * lda + c) = hp;
        *reinterpret_cast<uint2*>(Al + m * lda + c) = lp;
    }
}

// ================================================================================================
// Embedding gathers.  One wavefront per row; lane j copies elements 4j.. of each 256-wide slab.
// The model input of lane b at position p of a compress pass: its byte inside the chunk, 0 past its end.
__device__ __forceinline__ int byte_token(const uint8_t* bytes, int64_t stride, const int32_t* lens, int64_t b, int p,
                                          int V) {
    const int tok = (p < lens[b]) ? (int)bytes[b * stride + p] : 0;
    return tok < V ? tok : V - 1;  // bytes >= vocab are not codable; keep the gather in bounds
}

__global__ void __launch_bounds__(256) k_embed_bytes(const uint8_t* __restrict__ bytes, int64_t stride,
                                                    const int32_t* __restrict__ lens, int t0, int Tc,
                                                    int64_t rows, const float* __restrict__ emb, int d, int V,
                                                    float* __restrict__ x) {
    const int64_t m = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (m >= rows) return;
    const int64_t b = m / Tc;
    const int t = (int)(m - b * Tc);
    const int tok = byte_token(bytes, stride, lens, b, t0 + t, V);
    for (int c = 4 * lane; c < d; c += 256)
        *reinterpret_cast<float4*>(x + m * d + c) = *reinterpret_cast<const float4*>(emb + (int64_t)tok * d + c);
}

// Layer 0 of a full compress tile reads its input rows straight from the embedding table in the LN1 prologue of
// the mixer-input kernel (k_mixin, k_mixin512: template parameter EMB), which also writes them to x, the residual
// stream the feed-forward kernel adds to; the separate embedding pass (k_embed_bytes) and its HBM round trip are
// skipped.  Without EMB the kernels read x as written by an embedding pass or the previous layer, and ignore this.
struct EmbedIn {
    const uint8_t* bytes = nullptr;  // the group's bytes [lanes][stride]
    int64_t stride = 0;
    const int32_t* lens = nullptr;   // the group's chunk lengths
    const float* emb = nullptr;      // [V][d]
    float* xout = nullptr;           // x, where the gathered rows are written for the residual
    int t0 = 0, V = 0;               // the tile's first position; vocab
};

__global__ void __launch_bounds__(256) k_embed_tokens(const int32_t* __restrict__ tokens, int64_t tok_stride,
                                                     int t0, int Tc, int64_t rows, const float* __restrict__ emb,
                                                     int d, int V, float* __restrict__ x) {
    const int64_t m = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (m >= rows) return;
    const int64_t b = m / Tc;
    const int t = (int)(m - b * Tc);
    int tok = tokens[b * tok_stride + t0 + t];
    tok = tok < 0 ? 0 : (tok >= V ? V - 1 : tok);
    for (int c = 4 * lane; c < d; c += 256)
        *reinterpret_cast<float4*>(x + m * d + c) = *reinterpret_cast<const float4*>(emb + (int64_t)tok * d + c);
}

// ================================================================================================
// Depthwise causal conv (d_conv = 4) + bias + SiLU, per (lane, channel), sequential over the Tc positions
// of the launch (conv_point).  History = the 3 previous x values of the channel, [lane][3][di] in HBM
// between launches, as a ring: the input of absolute position p lives in slot p % 3, so the history of
// position p0 is slots p0 % 3 (x[p0-3]), (p0+1) % 3 (x[p0-2]), (p0+2) % 3 (x[p0-1]) and a one-position
// launch rewrites one slot only.  p0m3 = p0 % 3.
__global__ void __launch_bounds__(256) k_conv_silu(const float* __restrict__ xz, int64_t ldxz,
                                                  float* __restrict__ hist, const float* __restrict__ w,
                                                  const float* __restrict__ bias, float* __restrict__ xs,
                                                  int di, int Tc, int p0m3) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t b = blockIdx.y;
    if (c >= di) return;
    float* hb = hist + b * 3 * di;
    const int s1 = p0m3 == 2 ? 0 : p0m3 + 1, s2 = p0m3 == 0 ? 2 : p0m3 - 1;
    float h0 = hb[p0m3 * di + c], h1 = hb[s1 * di + c], h2 = hb[s2 * di + c];
    const float4 wv = *reinterpret_cast<const float4*>(w + 4 * c);
    const float bb = bias[c];
    for (int t = 0; t < Tc; ++t) {
        const int64_t m = b * Tc + t;
        const float x = xz[m * ldxz + c];
        xs[m * di + c] = conv_point(wv, bb, h0, h1, h2, x);
        h0 = h1; h1 = h2; h2 = x;
    }
    // h0, h1, h2 = inputs of positions p0+Tc-3 .. p0+Tc-1 (or older history, rewritten unchanged)
    const int e0 = (p0m3 + Tc) % 3, e1 = (e0 + 1) % 3, e2 = (e0 + 2) % 3;
    hb[e0 * di + c] = h0; hb[e1 * di + c] = h1; hb[e2 * di + c] = h2;
}

// ================================================================================================
// Decompress-step fusion of the conv + SiLU and x_proj (split-precision modes): one workgroup owns 16 lanes.
//   phase 1: conv_point for one position, x into LDS (and to xs for the scan), one history slot rewritten;
//   phase 2: x_proj on v_mfma_f32_16x16x32_bf16 with A split from LDS exactly as k_gemm_bf splits fp32 A
//            on load, the same product order (lo*hi, hi*lo, hi*hi) and ascending 32-wide K steps, one wave
//            per 16-column output fragment, so every output equals the standalone GEMM's bit for bit.
template <int NT>
__global__ void __launch_bounds__(256) k_convx_step(const float* __restrict__ xz, int64_t ldxz, float* __restrict__ hist,
                                                   const float* __restrict__ w, const float* __restrict__ bias,
                                                   float* __restrict__ xs, const uint16_t* __restrict__ Wh,
                                                   const uint16_t* __restrict__ Wl, float* __restrict__ dbc, int ldd,
                                                   int di, int B, int p0m3) {
    extern __shared__ float sX[];  // [16][di + 4]
    const int LDX = di + 4;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t b0 = (int64_t)blockIdx.x * 16;
    const int s1 = p0m3 == 2 ? 0 : p0m3 + 1, s2 = p0m3 == 0 ? 2 : p0m3 - 1;
    // History rows of lanes [b0, b0 + nb) through a range-checked buffer (rows past B read 0 and are not
    // written), non-temporal, all 16 lanes' loads in flight before the first use; rows past B take the last
    // lane's x and are not stored.  Offsets are formed per lane from an opaque channel index (not held).
    const int nb = (int)((B - b0) < 16 ? (B - b0) : 16);
    const __amdgpu_buffer_rsrc_t hr = buf_rsrc(hist + b0 * 3 * di, (uint32_t)nb * 3 * di * 4);
    for (int c = tid; c < di; c += 256) {
        const float4 wv = ldg_f4(G(w) + 4 * c);
        const float bb = G(bias)[c];
        float h0[16], h1[16], h2[16], xv[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            int cq = c;
            __asm__ volatile("" : "+v"(cq));
            const uint32_t o = (uint32_t)(r * 3 * di + cq) * 4;
            h0[r] = buf_ld1(hr, o + p0m3 * di * 4);
            h1[r] = buf_ld1(hr, o + s1 * di * 4);
            h2[r] = buf_ld1(hr, o + s2 * di * 4);
            xv[r] = G(xz)[(b0 + (r < nb ? r : nb - 1)) * ldxz + cq];
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            int cq = c;
            __asm__ volatile("" : "+v"(cq));
            const float y = conv_point(wv, bb, h0[r], h1[r], h2[r], xv[r]);
            if (r < nb) xs[(b0 + r) * di + cq] = y;
            sX[r * LDX + cq] = y;
            buf_st1(hr, (uint32_t)(r * 3 * di + p0m3 * di + cq) * 4, xv[r]);
        }
    }
    __syncthreads();
    if (wave * 16 >= ldd) return;  // ldd = r + 2N output columns: 48 (d 256) or 64 (d 512)
    const int i = lane & 15, kq = 8 * (lane >> 4);
    const int n = wave * 16 + i;
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int q = 0; q < di / XPROJ_KB; ++q) {
        floatx4 part = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k0 = XPROJ_KB * q; k0 < XPROJ_KB * (q + 1); k0 += 32) {
            const float* xa = &sX[i * LDX + k0 + kq];
            bf16x8 ah, al;
            split8(xa, ah, al);
            const bf16x8 bh = *reinterpret_cast<const bf16x8*>(Wh + (int64_t)n * di + k0 + kq);
            bf16x8 bl = bh;
            if constexpr (NT == 3) bl = *reinterpret_cast<const bf16x8*>(Wl + (int64_t)n * di + k0 + kq);
            part = mfma_split_step<NT>(part, ah, al, bh, bl);
        }
        acc = q == 0 ? part : acc + part;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t b = b0 + 4 * (lane >> 4) + r;
        if (b < B) dbc[b * ldd + wave * 16 + (lane & 15)] = acc[r];
    }
}

// x_proj over M rows in the split modes (compress tiles): one wavefront per 16 rows computes all NF output
// fragments, A = xs fp32 [M][di] split on load, W [N][K] bf16 parts.  Outputs follow the K-block fold of
// XPROJ_KB (P_q from zero over the two K steps of block q, then dbc = P_0 + P_1 + ...), like k_convx_step and
// the fused decode kernel, so a position's dbc row is the same in all three.  Row m of the output depends on
// row m of A only.
template <int NT, int NF>
__global__ void __launch_bounds__(256) k_xproj(const float* __restrict__ xs, int64_t M, int di,
                                              const uint16_t* __restrict__ Wh, const uint16_t* __restrict__ Wl,
                                              float* __restrict__ dbc, int ldd) {
    const int lane = threadIdx.x & 63;
    const int64_t m0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 16;
    if (m0 >= M) return;
    const int ar = lane & 15, kq = 8 * (lane >> 4);
    const bool ok = m0 + ar < M;
    const float* xr = xs + (m0 + ar) * di + kq;
    floatx4 acc[NF];
    for (int q = 0; q < di / XPROJ_KB; ++q) {
        floatx4 part[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f) part[f] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < XPROJ_KB / 32; ++s) {
            const int k0 = XPROJ_KB * q + 32 * s;
            float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (ok) {
                const float4 a0 = *reinterpret_cast<const float4*>(xr + k0);
                const float4 a1 = *reinterpret_cast<const float4*>(xr + k0 + 4);
                v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w; v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
            }
            bf16x8 ah, al;
            split8(v, ah, al);
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                const int64_t wo = (int64_t)(16 * f + ar) * di + k0 + kq;
                const bf16x8 bh = *reinterpret_cast<const bf16x8*>(Wh + wo);
                bf16x8 bl = bh;
                if constexpr (NT == 3) bl = *reinterpret_cast<const bf16x8*>(Wl + wo);
                part[f] = mfma_split_step<NT>(part[f], ah, al, bh, bl);
            }
        }
#pragma unroll
        for (int f = 0; f < NF; ++f) acc[f] = q == 0 ? part[f] : acc[f] + part[f];
    }
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = m0 + 4 * (lane >> 4) + r;
            if (row < M) dbc[row * ldd + 16 * f + ar] = acc[f][r];
        }
}

// x_proj in the fp32 mode for the layer-by-layer path: one wavefront per 16 rows computes all NF output fragments
// from xs [M][di] and the fp32 weight matrix W [N][di] (row-major, as in the weight blob), with the K-block fold of
// XPROJ_KB: P_q accumulates the four 16-K groups of channels 64 q .. 64 q + 63 from zero through
// v_mfma_f32_16x16x4_f32 (lane l supplies k = 16 g + 4 (l / 16) + j to the j-th MFMA of group g, as every fp32
// kernel does), then dbc = P_0 + P_1 + ....  A position's dbc row is therefore the one the fused fp32 compress
// (k_mixin<1>) and decode (k_fused_step<1, 512>) kernels compute.  Row m of the output depends on row m of xs only.
template <int NF>
__global__ void __launch_bounds__(256) k_xproj_f32(const float* __restrict__ xs, int64_t M, int di,
                                                  const float* __restrict__ W, float* __restrict__ dbc, int ldd) {
    const int lane = threadIdx.x & 63;
    const int64_t m0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 16;
    if (m0 >= M) return;
    const int ar = lane & 15, kq = 4 * (lane >> 4);
    const bool ok = m0 + ar < M;
    floatx4 acc[NF];
    for (int q = 0; q < di / XPROJ_KB; ++q) {
        floatx4 part[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f) part[f] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int g = 0; g < XPROJ_KB / 16; ++g) {
            const int k0 = XPROJ_KB * q + 16 * g + kq;
            float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
            if (ok) a = *reinterpret_cast<const float4*>(xs + (m0 + ar) * di + k0);
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                const float4 b = *reinterpret_cast<const float4*>(W + (int64_t)(16 * f + ar) * di + k0);
                part[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, part[f], 0, 0, 0);
                part[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, part[f], 0, 0, 0);
                part[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, part[f], 0, 0, 0);
                part[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, part[f], 0, 0, 0);
            }
        }
#pragma unroll
        for (int f = 0; f < NF; ++f) acc[f] = q == 0 ? part[f] : acc[f] + part[f];
    }
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = m0 + 4 * (lane >> 4) + r;
            if (row < M) dbc[row * ldd + 16 * f + ar] = acc[f][r];
        }
}

// ================================================================================================
// Feed-forward half of a block in one kernel (split modes, d_model 256, d_ff 1024), for row tiles:
//   x <- x + FF2(GELU(FF1(LN2(mm))))        (model.py:60-65: Linear -> GELU -> Linear, then the block residual)
// A workgroup owns 64 rows.  LN2 of its rows goes to LDS as the split operand; then, per 64-wide chunk of the
// hidden layer, FF1 (+bias, GELU, split) writes the chunk to LDS and FF2 accumulates it into registers, so the
// hidden activations never leave the chip (the unfused path writes and reads back 4 KiB of them per row).
// Arithmetic per output is that of the tiled GEMMs and of the fused decode kernel: LN by ln_stats_row /
// ln_apply / split2; FF1 outputs accumulate their 8 K steps in ascending order through mfma_split_step (its
// transposed form, same value) then epi_value<GELU>; FF2 outputs accumulate all 32 K steps in ascending order (chunk by chunk), then
// x + epi_value<RESID>.  So the rows equal those of the layer-by-layer path bit for bit.
// LDS: A [64][256] (hi, lo) and H [64][64] (hi, lo), bf16, 16-byte chunks XOR-swizzled by row so that 16-row
// fragment reads touch every bank once; 80 KB, two workgroups per CU.
namespace ffn {
constexpr int BM = 64, D = 256, DF = 1024, HC = 64;
__device__ __forceinline__ int a_off(int r, int k) { return r * D + ((((k >> 3) ^ r) & 15) | ((k >> 3) & 16)) * 8 + (k & 7); }
__device__ __forceinline__ int h_off(int r, int k) { return r * HC + (((k >> 3) ^ (r >> 1)) & 7) * 8 + (k & 7); }
}  // namespace ffn

// 512 threads (8 waves), two workgroups (4 waves per SIMD) per CU, at most 128 VGPRs:
//   FF1: wave w computes rows 32 (w & 1) .. + 31 x hidden units 16 (w >> 1) .. + 15 of the chunk, the W1 block
//        as the A operand (mfma_split_step_t), so a lane's 4 GELU outputs are consecutive hidden units (one
//        8-byte store per part); each W1 block is read by two waves.
//   FF2: wave w owns outputs 32 w .. + 31 (2 fragments) for all 64 rows.
// Per chunk a wave streams 12 weight blocks through one ring of R register slots, in the order it uses them:
// 8 W1 blocks (K step s), then 4 W2 blocks (fragment 2 w + q % 2, K step 2 c + q / 2).  Block i goes to slot
// i % R and is reloaded with block i + R right after its use, running on into the next chunk, so R blocks
// are always in flight; pin_loads keeps each reload where it is issued.  (4 waves per SIMD instead of 2:
// 6% faster than the 4-wave form with 64 x 16 FF1 tiles, which reads each W1 block once.)
// OUTP: the out_proj GEMM runs first, inside this kernel: mm = y . W_out^T + b_out from the scan's split output
// y [rows][512] (hi, lo), read in two K chunks of 256 staged through the LDS operand buffer, each output
// accumulating its 16 K steps in ascending order through mfma_split_step (as the out_proj GEMM does); mm then
// stays on chip (fp32 in the operand buffer) for LN2, instead of a round trip through HBM.  Wave w owns
// out_proj outputs 32 w .. + 31 of all 64 rows; its 32 W_out blocks stream through a 4-slot ring.
template <int NT, bool OUTP>
__global__ void __launch_bounds__(512, 4) k_ffn(const float* __restrict__ mm, const float* __restrict__ ln_w,
                                                const float* __restrict__ ln_b, const uint16_t* __restrict__ W1p,
                                                const float* __restrict__ b1, const uint16_t* __restrict__ W2p,
                                                const float* __restrict__ b2, float* __restrict__ x, int64_t M,
                                                const uint16_t* __restrict__ yh, const uint16_t* __restrict__ yl,
                                                const uint16_t* __restrict__ Wop, const float* __restrict__ bo) {
    using namespace ffn;
    __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * D];
    __shared__ __attribute__((aligned(16))) uint16_t sH[2][BM * HC];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const int rows = (int)((M - m0) < BM ? (M - m0) : BM);
    // LN2 of one row held by one wave (lane j: elements 4j .. 4j + 3) into the split operand
    auto ln2_store = [&](int r, const float (&v)[4], float4 wv, float4 bv) {
        float mu, rs;
        ln_stats_row<1>(v, mu, rs);
        const float y[4] = {ln_apply(v[0], mu, rs, wv.x, bv.x), ln_apply(v[1], mu, rs, wv.y, bv.y),
                            ln_apply(v[2], mu, rs, wv.z, bv.z), ln_apply(v[3], mu, rs, wv.w, bv.w)};
        if constexpr (NT == 1) {
            const int k = 4 * lane;
            *reinterpret_cast<float4*>(&sA[f32_lo(k)][a_off(r, f32_col(k))]) = make_float4(y[0], y[1], y[2], y[3]);
        } else {
            uint2 hp, lp;
            split4(y[0], y[1], y[2], y[3], hp, lp);
            const int o = a_off(r, 4 * lane);
            *reinterpret_cast<uint2*>(&sA[0][o]) = hp;
            *reinterpret_cast<uint2*>(&sA[1][o]) = lp;
        }
    };
    if constexpr (OUTP) {
        constexpr int KO = 2 * D, KC = D, NKS = KO / 32, BLKO = two_part_blocks<NT>() ? 1024 : 512, RO = 4;
        const __amdgpu_buffer_rsrc_t wop = wbuf(Wop);
        u32x4 oh[RO], ol[RO];
        // block i (W_out fragment 2 wave + i % 2, K step i / 2) into ring slot i % RO
        auto issue_o = [&](int i) {
            const uint32_t bo = (uint32_t)(((2 * wave + (i & 1)) * NKS + (i >> 1)) * BLKO * 2);
            oh[i % RO] = wbuf_ld16(wop, lane * 16, bo);
            ol[i % RO] = oh[i % RO];
            if constexpr (two_part_blocks<NT>()) ol[i % RO] = wbuf_ld16(wop, lane * 16, bo + 1024);
        };
#pragma unroll
        for (int i = 0; i < RO; ++i) issue_o(i);
        floatx4 macc[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) macc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
        // y rows past M read 0 (buffer range check).  NT = 1: y is fp32 [rows][512] at yh (yl unused).
        const __amdgpu_buffer_rsrc_t ryh = buf_rsrc(yh + m0 * KO * (NT == 1 ? 2 : 1), (uint32_t)rows * KO * (NT == 1 ? 4 : 2));
        const __amdgpu_buffer_rsrc_t ryl = NT == 1 ? ryh : buf_rsrc(yl + m0 * KO, (uint32_t)rows * KO * 2);
#pragma unroll 1
        for (int q = 0; q < KO / KC; ++q) {
            if constexpr (NT == 1) {
                // stage y[:, 256 q .. + 255] (fp32, in the split operand's layout): 8 x 16 B per thread, 2 in
                // flight (more spill registers: the kernel is at its 128-register limit)
#pragma unroll 2
                for (int e = 0; e < (BM * KC / 4) / 512; ++e) {
                    const int idx = e * 512 + tid, r = idx / (KC / 4), k = (idx % (KC / 4)) * 4;
                    const uint32_t off = (uint32_t)((r * KO + KC * q + k) * 4);
                    *reinterpret_cast<u32x4*>(&sA[f32_lo(k)][a_off(r, f32_col(k))]) = buf_ld16(ryh, off);
                }
            } else {
                // stage y[:, 256 q .. + 255] (hi, lo): 4 x 16 B per array per thread
#pragma unroll
                for (int e = 0; e < (BM * KC / 8) / 512; ++e) {
                    const int idx = e * 512 + tid, r = idx / (KC / 8), k = (idx % (KC / 8)) * 8;
                    const uint32_t off = (uint32_t)((r * KO + KC * q + k) * 2);
                    *reinterpret_cast<u32x4*>(&sA[0][a_off(r, k)]) = buf_ld16(ryh, off);
                    *reinterpret_cast<u32x4*>(&sA[1][a_off(r, k)]) = buf_ld16(ryl, off);
                }
            }
            __syncthreads();
            int lq = lane;  // LDS addresses formed per chunk (see k_head_xq)
            __asm__ volatile("" : "+v"(lq));
            const int arq = lq & 15, kqq = 8 * (lq >> 4);
#pragma unroll
            for (int s = 0; s < KC / 32; ++s) {
                bf16x8 ah[4], al[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int o = a_off(16 * i + arq, 32 * s + kqq);
                    ah[i] = *reinterpret_cast<const bf16x8*>(&sA[0][o]);
                    al[i] = *reinterpret_cast<const bf16x8*>(&sA[1][o]);
                }
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int bi = 2 * ((KC / 32) * q + s) + j;  // block index over the whole K
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        macc[i][j] = mfma_split_step<NT>(macc[i][j], ah[i], al[i], __builtin_bit_cast(bf16x8, oh[bi % RO]),
                                                         __builtin_bit_cast(bf16x8, ol[bi % RO]));
                    if (bi + RO < 2 * NKS) issue_o(bi + RO);
                    pin_loads();
                }
            }
            __syncthreads();  // the next chunk (or mm) rewrites the operand buffer
        }
        // mm (+ bias) as fp32 rows of 256 in the operand buffer
        float* sM = reinterpret_cast<float*>(&sA[0][0]);
        const int ar = lane & 15, m_of = 4 * (lane >> 4);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = 16 * (2 * wave + j) + ar;
            const float bias = G(bo)[col];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) sM[(16 * i + m_of + r) * D + col] = epi_value<EPI_BIAS>(macc[i][j][r], bias);
        }
        __syncthreads();
        // LN2 of this wave's 8 rows: all read before any split is written over the fp32 rows
        float v[8][4];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 u = *reinterpret_cast<const float4*>(&sM[(8 * wave + q) * D + 4 * lane]);
            v[q][0] = u.x; v[q][1] = u.y; v[q][2] = u.z; v[q][3] = u.w;
        }
        const float4 wv = ldg_f4(G(ln_w) + 4 * lane), bv = ldg_f4(G(ln_b) + 4 * lane);
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 8; ++q) ln2_store(8 * wave + q, v[q], wv, bv);
    } else {
        const __amdgpu_buffer_rsrc_t rm = buf_rsrc(mm + m0 * D, (uint32_t)rows * D * 4);
        const float4 wv = ldg_f4(G(ln_w) + 4 * lane), bv = ldg_f4(G(ln_b) + 4 * lane);
#pragma unroll 4
        for (int q = 0; q < BM / 8; ++q) {
            const int r = 8 * wave + q;
            const u32x4 u = buf_ld16(rm, (uint32_t)((r * D + 4 * lane) * 4));
            const float v[4] = {__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w)};
            ln2_store(r, v, wv, bv);
        }
    }
    __syncthreads();
    const int ar = lane & 15, kq = 8 * (lane >> 4), m_of = 4 * (lane >> 4);
    constexpr int BLK = two_part_blocks<NT>() ? 1024 : 512;
    const __amdgpu_buffer_rsrc_t w1p = wbuf(W1p), w2p = wbuf(W2p);
    const int rh = wave & 1, cf = wave >> 1;
    constexpr int NBC = 12, R = 4;
    static_assert(NBC % R == 0, "ring slots divide the blocks of a chunk");
    u32x4 rhh[R], rll[R];
    auto issue = [&](int c, int i) {
        const int blk = i < 8 ? (4 * c + cf) * (D / 32) + i
                              : (2 * wave + ((i - 8) & 1)) * (DF / 32) + 2 * c + ((i - 8) >> 1);
        const __amdgpu_buffer_rsrc_t wr = i < 8 ? w1p : w2p;
        rhh[i % R] = wbuf_ld16(wr, lane * 16, (uint32_t)(blk * BLK * 2));
        rll[i % R] = rhh[i % R];
        if constexpr (two_part_blocks<NT>()) rll[i % R] = wbuf_ld16(wr, lane * 16, (uint32_t)(blk * BLK * 2 + 1024));
    };
    auto refill = [&](int c, int cn, int i) {
        if (i + R < NBC) issue(c, i + R);
        else issue(cn, i + R - NBC);
    };
    floatx4 out[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) out[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < R; ++i) issue(0, i);
#pragma unroll 1
    for (int c = 0; c < DF / HC; ++c) {
        const int cn = c + 1 < DF / HC ? c + 1 : c;
        const float4 bias = ldg_f4(G(b1) + HC * c + 16 * cf + m_of);
        floatx4 hacc[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) hacc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            bf16x8 ah[2], al[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int o = a_off(32 * rh + 16 * i + ar, 32 * s + kq);
                ah[i] = *reinterpret_cast<const bf16x8*>(&sA[0][o]);
                al[i] = *reinterpret_cast<const bf16x8*>(&sA[1][o]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
                hacc[i] = mfma_split_step_t<NT>(hacc[i], ah[i], al[i], __builtin_bit_cast(bf16x8, rhh[s % R]),
                                                __builtin_bit_cast(bf16x8, rll[s % R]));
            refill(c, cn, s);
            pin_loads();
        }
        {
            const float bv[4] = {bias.x, bias.y, bias.z, bias.w};
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                float g[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) g[r] = epi_value<EPI_GELU>(hacc[i][r], bv[r]);
                if constexpr (NT == 1) {
                    const int k = 16 * cf + m_of;
                    *reinterpret_cast<float4*>(&sH[f32_lo(k)][h_off(32 * rh + 16 * i + ar, f32_col(k))]) =
                        make_float4(g[0], g[1], g[2], g[3]);
                } else {
                    uint2 hp, lp;
                    split4(g[0], g[1], g[2], g[3], hp, lp);
                    const int o = h_off(32 * rh + 16 * i + ar, 16 * cf + m_of);
                    *reinterpret_cast<uint2*>(&sH[0][o]) = hp;
                    *reinterpret_cast<uint2*>(&sH[1][o]) = lp;
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            bf16x8 ah[4], al[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int o = h_off(16 * i + ar, 32 * t + kq);
                ah[i] = *reinterpret_cast<const bf16x8*>(&sH[0][o]);
                al[i] = *reinterpret_cast<const bf16x8*>(&sH[1][o]);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int bi = 8 + 2 * t + j;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    out[i][j] = mfma_split_step<NT>(out[i][j], ah[i], al[i], __builtin_bit_cast(bf16x8, rhh[bi % R]),
                                                    __builtin_bit_cast(bf16x8, rll[bi % R]));
                refill(c, cn, bi);
                pin_loads();
            }
        }
        __syncthreads();
    }
    // residual: every value read before any is written (a read after a write to the same buffer would wait for
    // that write, one memory round trip per value)
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x + m0 * D, (uint32_t)rows * D * 4);
    float res[2][4][4];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t o = (uint32_t)(((16 * i + m_of + r) * D + 16 * (2 * wave + j) + ar) * 4);
                res[j][i][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, o, 0, 0));
            }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int col = 16 * (2 * wave + j) + ar;
        const float bias = G(b2)[col];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t o = (uint32_t)(((16 * i + m_of + r) * D + col) * 4);
                __builtin_amdgcn_raw_buffer_store_b32(
                    __builtin_bit_cast(uint32_t, res[j][i][r] + epi_value<EPI_RESID>(out[i][j][r], bias)), rx, o, 0, 0);
            }
    }
}

// ================================================================================================
// The same feed-forward half for d_model 512 (d_ff 2048; configs[4]'s shape):
//   x <- x + FF2(GELU(FF1(LN2(mm))))
// A workgroup of 512 threads owns 64 rows (one workgroup per CU: the LN2 operand is 128 KB).  Per chunk of the
// hidden layer (64 units wide, 128 with bf16 weights): FF1 (+bias, GELU, split) into LDS, then FF2 accumulates
// the chunk into registers, so the hidden activations never leave the chip.  The arithmetic of every value is that of the layer-by-layer path
// (ln_stats_row / ln_apply / split2; FF1 outputs accumulate their 16 K steps in ascending order through
// mfma_split_step_t, then epi_value<GELU>; FF2 outputs accumulate all 64 K steps in ascending order, chunk by
// chunk, then x + epi_value<RESID>), so rows equal those of the GEMM kernels bit for bit.  Used by the compress
// tiles (64 positions of one lane) and by the per-layer decode step (64 lanes of one position).
//   FF1: wave w computes rows 32 (w & 1) .. + 31 x FG fragments of 16 hidden units of the chunk (fragments
//        FG (w >> 1) ..; FG = ffn_groups), the W1 block as the MFMA A operand (a lane's 4 outputs are 4
//        consecutive hidden units, one 8-byte store per part).  With bf16 weights the LN2 operand fragments of the
//        next K step are read before the current step's MFMAs, with scheduling fences around each step (without
//        them the compiler moves each MFMA up to its own operand read, and every MFMA waits for LDS).
//   FF2: wave w owns outputs 64 w .. + 63 (4 fragments) of all 64 rows: 16 accumulators.
// Per chunk a wave uses 24 FG weight blocks (16 FG of W1, then 8 FG of W2) through a ring of R register slots in
// use order, running on into the next chunk, so R blocks are always in flight.
namespace ffn5 {
constexpr int BM = 64, D = 512, DF = 2048, HC = 64;
// 16-byte chunks XOR-swizzled by row (low 4 bits of the chunk index), so 16-row fragment reads spread over banks
__device__ __forceinline__ int a_off(int r, int k) { return r * D + (((k >> 3) ^ (r & 15)) << 3) + (k & 7); }
// the hidden chunk [64][HW] (HW = 64: 8 chunks of 16 bytes per row, swizzled by row / 2; HW = 128: 16 per row,
// swizzled by row)
template <int HW>
__device__ __forceinline__ int h_off(int r, int k) {
    if constexpr (HW == 64) return r * HW + (((k >> 3) ^ (r >> 1)) & 7) * 8 + (k & 7);
    else return r * HW + (((k >> 3) ^ r) & 15) * 8 + (k & 7);
}
// W1 fragments per wave and hidden chunk: 2 with bf16 weights (chunks of 128 hidden units: each LN2 operand
// fragment read from LDS feeds two weight blocks), 1 with bf16x3 weights (no registers to spare)
template <int NT>
constexpr int ffn_groups() { return NT == 2 ? 2 : 1; }
}  // namespace ffn5

// OUTP: the out_proj GEMM runs first, inside this kernel (decode step and compress tiles at d_model 512): mm =
// y . W_out^T + b_out from the scan's split output y [rows][1024] (hi, lo), read in two K chunks of 512 staged
// through the LDS operand buffer, each output accumulating its 32 K steps in ascending order through
// mfma_split_step (as the out_proj GEMM does); mm then stays on chip (fp32 in the operand buffer) for LN2.
// Wave w owns out_proj outputs 64 w .. + 63 of all 64 rows; its W_out blocks stream through an 8-slot ring.
template <int NT, bool OUTP>
__global__ void __launch_bounds__(512, 2) k_ffn512(const float* __restrict__ mm, const float* __restrict__ ln_w,
                                                   const float* __restrict__ ln_b, const uint16_t* __restrict__ W1p,
                                                   const float* __restrict__ b1, const uint16_t* __restrict__ W2p,
                                                   const float* __restrict__ b2, float* __restrict__ x, int64_t M,
                                                   const uint16_t* __restrict__ yh, const uint16_t* __restrict__ yl,
                                                   const uint16_t* __restrict__ Wop, const float* __restrict__ bo) {
    using namespace ffn5;
    __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * D];
    __shared__ __attribute__((aligned(16))) uint16_t sH[2][BM * HC * ffn_groups<NT>()];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const int rows = (int)((M - m0) < BM ? (M - m0) : BM);
    const float4 w0 = ldg_f4(G(ln_w) + 4 * lane), w1 = ldg_f4(G(ln_w) + 256 + 4 * lane);
    const float4 c0 = ldg_f4(G(ln_b) + 4 * lane), c1 = ldg_f4(G(ln_b) + 256 + 4 * lane);
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    const float bv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    // LN2 of one row held by one wave (lane j: elements 4j.. and 256 + 4j..) into the split operand
    auto ln2_store = [&](int r, const float (&v)[8]) {
        float mu, rs;
        ln_stats_row<2>(v, mu, rs);
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = ln_apply(v[i], mu, rs, wv[i], bv[i]);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint2 hp, lp;
            split4(y[4 * h], y[4 * h + 1], y[4 * h + 2], y[4 * h + 3], hp, lp);
            const int o = a_off(r, 256 * h + 4 * lane);
            *reinterpret_cast<uint2*>(&sA[0][o]) = hp;
            *reinterpret_cast<uint2*>(&sA[1][o]) = lp;
        }
    };
    if constexpr (OUTP) {
        constexpr int KO = 2 * D, KC = D, NKS = KO / 32, BLKO = (NT == 3) ? 1024 : 512, RO = 8;
        const int ar = lane & 15, kq = 8 * (lane >> 4), m_of = 4 * (lane >> 4);
        const gptr<uint16_t> wop = G(Wop);
        u32x4 oh[RO], ol[RO];
        // block i (W_out fragment 4 wave + i % 4, K step i / 4) into ring slot u (= i % RO, passed as a constant)
        auto issue_o = [&](int u, int i) {
            const gptr<uint16_t> q = wop + ((int64_t)(4 * wave + (i & 3)) * NKS + (i >> 2)) * BLKO + lane * 8;
            oh[u] = ldg16(q);
            ol[u] = oh[u];
            if constexpr (NT == 3) ol[u] = ldg16(q + 512);
        };
#pragma unroll
        for (int i = 0; i < RO; ++i) issue_o(i, i);
        floatx4 macc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) macc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
        // y rows past M read 0 (buffer range check)
        const __amdgpu_buffer_rsrc_t ryh = buf_rsrc(yh + m0 * KO, (uint32_t)rows * KO * 2);
        const __amdgpu_buffer_rsrc_t ryl = buf_rsrc(yl + m0 * KO, (uint32_t)rows * KO * 2);
#pragma unroll 1
        for (int q = 0; q < KO / KC; ++q) {
            // stage y[:, 512 q .. + 511] (hi, lo): 8 x 16 B per array per thread
#pragma unroll
            for (int e = 0; e < (BM * KC / 8) / 512; ++e) {
                const int idx = e * 512 + tid, r = idx / (KC / 8), k = (idx % (KC / 8)) * 8;
                const uint32_t off = (uint32_t)((r * KO + KC * q + k) * 2);
                *reinterpret_cast<u32x4*>(&sA[0][a_off(r, k)]) = buf_ld16(ryh, off);
                *reinterpret_cast<u32x4*>(&sA[1][a_off(r, k)]) = buf_ld16(ryl, off);
            }
            __syncthreads();
#pragma unroll 2
            for (int s = 0; s < KC / 32; ++s) {
                bf16x8 ah[4], al[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int o = a_off(16 * i + ar, 32 * s + kq);
                    ah[i] = *reinterpret_cast<const bf16x8*>(&sA[0][o]);
                    al[i] = *reinterpret_cast<const bf16x8*>(&sA[1][o]);
                }
                const int sg = (KC / 32) * q + s;  // K step over the whole K
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int bi = 4 * sg + j, u = (4 * s + j) % RO;  // 4 sg = 64 q + 4 s: same slot as bi % RO
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        macc[i][j] = mfma_split_step<NT>(macc[i][j], ah[i], al[i], __builtin_bit_cast(bf16x8, oh[u]),
                                                         __builtin_bit_cast(bf16x8, ol[u]));
                    if (bi + RO < 4 * NKS) issue_o(u, bi + RO);
                    pin_loads();
                }
            }
            __syncthreads();  // the next chunk (or mm) rewrites the operand buffer
        }
        // mm (+ bias) as fp32 rows of 512 in the operand buffer
        float* sM = reinterpret_cast<float*>(&sA[0][0]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = 16 * (4 * wave + j) + ar;
            const float bias = G(bo)[col];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) sM[(16 * i + m_of + r) * D + col] = epi_value<EPI_BIAS>(macc[i][j][r], bias);
        }
        __syncthreads();
        // LN2 of this wave's 8 rows: all read before any split is written over the fp32 rows
        float v[8][8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int r = 8 * wave + q;
            const float4 u0 = *reinterpret_cast<const float4*>(&sM[r * D + 4 * lane]);
            const float4 u1 = *reinterpret_cast<const float4*>(&sM[r * D + 256 + 4 * lane]);
            v[q][0] = u0.x; v[q][1] = u0.y; v[q][2] = u0.z; v[q][3] = u0.w;
            v[q][4] = u1.x; v[q][5] = u1.y; v[q][6] = u1.z; v[q][7] = u1.w;
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 8; ++q) ln2_store(8 * wave + q, v[q]);
    } else {
        // LN2 of 8 rows per wave; rows past M read 0 (buffer range check) and are never stored
        const __amdgpu_buffer_rsrc_t rm = buf_rsrc(mm + m0 * D, (uint32_t)rows * D * 4);
#pragma unroll 2
        for (int q = 0; q < BM / 8; ++q) {
            const int r = 8 * wave + q;
            const u32x4 u0 = buf_ld16(rm, (uint32_t)((r * D + 4 * lane) * 4));
            const u32x4 u1 = buf_ld16(rm, (uint32_t)((r * D + 256 + 4 * lane) * 4));
            const float v[8] = {__uint_as_float(u0.x), __uint_as_float(u0.y), __uint_as_float(u0.z), __uint_as_float(u0.w),
                                __uint_as_float(u1.x), __uint_as_float(u1.y), __uint_as_float(u1.z), __uint_as_float(u1.w)};
            ln2_store(r, v);
        }
    }
    __syncthreads();
    const int ar = lane & 15, kq = 8 * (lane >> 4), m_of = 4 * (lane >> 4);
    constexpr int BLK = (NT == 3) ? 1024 : 512;
    const gptr<uint16_t> w1p = G(W1p), w2p = G(W2p);
    const int rh = wave & 1, cf = wave >> 1;
    constexpr int FG = ffn_groups<NT>(), HW = FG * HC, NB1 = D / 32, NF1 = FG * NB1, NBC = NF1 + HW / 8, R = 6;
    static_assert(NBC % R == 0, "ring slots divide the blocks of a chunk");
    u32x4 rhh[R], rll[R];
    // block i of chunk c: i < NF1: W1 fragment (4 c + cf) FG + i % FG, K step i / FG; else W2 fragment
    // 4 wave + (i - NF1) % 4, K step (HW / 32) c + (i - NF1) / 4
    auto issue = [&](int c, int i) {
        const int64_t blk = i < NF1 ? (int64_t)((4 * c + cf) * FG + i % FG) * (D / 32) + i / FG
                                    : (int64_t)(4 * wave + ((i - NF1) & 3)) * (DF / 32) + (HW / 32) * c + ((i - NF1) >> 2);
        const gptr<uint16_t> q = (i < NF1 ? w1p : w2p) + blk * BLK + lane * 8;
        rhh[i % R] = ldg16(q);
        rll[i % R] = rhh[i % R];
        if constexpr (NT == 3) rll[i % R] = ldg16(q + 512);
    };
    auto refill = [&](int c, int cn, int i) {
        if (i + R < NBC) issue(c, i + R);
        else issue(cn, i + R - NBC);
    };
    floatx4 out[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) out[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < R; ++i) issue(0, i);
#pragma unroll 1
    for (int c = 0; c < DF / HW; ++c) {
        const int cn = c + 1 < DF / HW ? c + 1 : c;
        float4 bias[FG];
#pragma unroll
        for (int g = 0; g < FG; ++g) bias[g] = ldg_f4(G(b1) + HW * c + 16 * (FG * cf + g) + m_of);
        floatx4 hacc[FG][2];
#pragma unroll
        for (int g = 0; g < FG; ++g)
#pragma unroll
            for (int i = 0; i < 2; ++i) hacc[g][i] = floatx4{0.f, 0.f, 0.f, 0.f};
        // the LN2 operand fragments of K step s into register slot u; with bf16 weights (NT 2) one K step ahead of
        // their MFMAs, so the LDS read latency is not exposed at every step (NT 3 has no registers to spare)
        constexpr int AS = NT == 2 ? 2 : 1;
        bf16x8 ah[AS][2], al[AS][2];
        auto lda = [&](int s, int u) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int o = a_off(32 * rh + 16 * i + ar, 32 * s + kq);
                ah[u][i] = *reinterpret_cast<const bf16x8*>(&sA[0][o]);
                al[u][i] = *reinterpret_cast<const bf16x8*>(&sA[1][o]);
            }
        };
        if constexpr (AS == 2) lda(0, 0);
#pragma unroll
        for (int s = 0; s < NB1; ++s) {
            if constexpr (AS == 2) {
                if (s + 1 < NB1) lda(s + 1, (s + 1) & 1);
                __builtin_amdgcn_sched_barrier(0);
            } else {
                lda(s, 0);
            }
            const int u = AS == 2 ? (s & 1) : 0;
#pragma unroll
            for (int g = 0; g < FG; ++g) {
                const int bi = FG * s + g;
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    hacc[g][i] = mfma_split_step_t<NT>(hacc[g][i], ah[u][i], al[u][i],
                                                       __builtin_bit_cast(bf16x8, rhh[bi % R]),
                                                       __builtin_bit_cast(bf16x8, rll[bi % R]));
                refill(c, cn, bi);
            }
            pin_loads();
            // nothing crosses a step boundary or the reads above: without the fences the scheduler moves each step's
            // MFMAs up to their operand reads, and the reads are back in front of their uses
            if constexpr (AS == 2) __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int g = 0; g < FG; ++g) {
            const float bv[4] = {bias[g].x, bias[g].y, bias[g].z, bias[g].w};
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                float h[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) h[r] = epi_value<EPI_GELU>(hacc[g][i][r], bv[r]);
                uint2 hp, lp;
                split4(h[0], h[1], h[2], h[3], hp, lp);
                const int o = h_off<HW>(32 * rh + 16 * i + ar, 16 * (FG * cf + g) + m_of);
                *reinterpret_cast<uint2*>(&sH[0][o]) = hp;
                *reinterpret_cast<uint2*>(&sH[1][o]) = lp;
            }
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < HW / 32; ++t) {
            bf16x8 ah[4], al[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int o = h_off<HW>(16 * i + ar, 32 * t + kq);
                ah[i] = *reinterpret_cast<const bf16x8*>(&sH[0][o]);
                al[i] = *reinterpret_cast<const bf16x8*>(&sH[1][o]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int bi = NF1 + 4 * t + j;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    out[i][j] = mfma_split_step<NT>(out[i][j], ah[i], al[i], __builtin_bit_cast(bf16x8, rhh[bi % R]),
                                                    __builtin_bit_cast(bf16x8, rll[bi % R]));
                refill(c, cn, bi);
                pin_loads();
            }
        }
        __syncthreads();
    }
    // residual: every value read before any is written (as in k_ffn)
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x + m0 * D, (uint32_t)rows * D * 4);
    float res[4][4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t o = (uint32_t)(((16 * i + m_of + r) * D + 16 * (4 * wave + j) + ar) * 4);
                res[j][i][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, o, 0, 0));
            }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int col = 16 * (4 * wave + j) + ar;
        const float bias = G(b2)[col];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t o = (uint32_t)(((16 * i + m_of + r) * D + col) * 4);
                __builtin_amdgcn_raw_buffer_store_b32(
                    __builtin_bit_cast(uint32_t, res[j][i][r] + epi_value<EPI_RESID>(out[i][j][r], bias)), rx, o, 0, 0);
            }
    }
}

// ================================================================================================
// Input half of the mixer in one kernel (split modes, d_model 256, compress tiles of 64 positions):
//   LN1 -> in_proj (+bias) -> z to HBM; x -> causal conv + SiLU over the 64 positions -> xs to HBM ->
//   x_proj -> dbc to HBM; the conv history ring of the lane advanced by 64 positions.
// A workgroup owns one lane's tile (rows b*64 .. b*64 + 63, positions p0 .. p0 + 63).  LN1 output is the split
// operand in LDS (as in k_ffn).  in_proj runs in 64-column chunks (each wave 16 columns x all 64 rows, the
// fragment-packed weight block as the MFMA A operand, through a register ring running on across chunks; a
// lane's 4 outputs are 4 consecutive columns of one row): the 8 z chunks are stored as they finish; each
// x chunk goes through LDS for the conv over time (the conv output, split, then replaces it in place) and
// into x_proj's partial over those 64 channels, which is exactly x_proj's K block, folded into dbc in
// registers (dbc = P_0 + P_1 + ...).  Arithmetic per value is that of the layer-by-layer kernels (ln_*,
// mfma_split_step, epi_value, conv_point, split2), so outputs equal theirs bit for bit.
namespace mixin {
constexpr int BM = 64, D = 256, DI = 512, CH = 64, FW = 48;
__device__ __forceinline__ int x_off(int r, int k) { return r * CH + (((k >> 3) ^ (r >> 1)) & 7) * 8 + (k & 7); }
// fp32 x chunk [64][64]: 16-byte groups XOR-swizzled by row, so both the in_proj stores (a lane's 4 columns, 16
// rows per instruction) and the conv's column reads (64 channels of one row) are free of bank conflicts
__device__ __forceinline__ int sx_off(int r, int c) { return r * CH + ((((c >> 2) ^ r) & 15) << 2) + (c & 3); }
}  // namespace mixin

template <int NT, bool EMB>
__global__ void __launch_bounds__(256, 2) k_mixin(const float* __restrict__ x, const float* __restrict__ ln_w,
                                                 const float* __restrict__ ln_b, const uint16_t* __restrict__ Wip,
                                                 const float* __restrict__ bin, const float* __restrict__ conv_w,
                                                 const float* __restrict__ conv_b, const uint16_t* __restrict__ Wxp,
                                                 float* __restrict__ xz, float* __restrict__ xs,
                                                 float* __restrict__ dbc, float* __restrict__ hist, int p0m3,
                                                 EmbedIn e) {
    using namespace mixin;
    constexpr int BLK = two_part_blocks<NT>() ? 1024 : 512;
    __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * D];  // LN1 output (hi, lo)
    __shared__ __attribute__((aligned(16))) float sX[BM * CH];        // x chunk fp32; then its conv output split
    uint16_t* sXh = reinterpret_cast<uint16_t*>(sX);
    uint16_t* sXl = sXh + BM * CH;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t b = blockIdx.x, m0 = b * BM;
    // ---- LN1 (layer 0 of a compress tile: of the embedding rows, which are also written to x at the end; lane q
    //      of a wave reads the token of its row q, handed to every lane by readlane)
    const int tokv = EMB ? byte_token(e.bytes, e.stride, e.lens, b, e.t0 + 16 * wave + (lane & 15), e.V) : 0;
    {
        const float4 wv = ldg_f4(G(ln_w) + 4 * lane), bv = ldg_f4(G(ln_b) + 4 * lane);
#pragma unroll 4
        for (int q = 0; q < BM / 4; ++q) {
            const int r = 16 * wave + q;
            float4 u;
            if constexpr (EMB) u = ldg_f4(G(e.emb) + (int64_t)__builtin_amdgcn_readlane(tokv, q) * D + 4 * lane);
            else u = ldg_f4(G(x) + (m0 + r) * D + 4 * lane);
            const float v[4] = {u.x, u.y, u.z, u.w};
            float mu, rs;
            ln_stats_row<1>(v, mu, rs);
            const float y[4] = {ln_apply(v[0], mu, rs, wv.x, bv.x), ln_apply(v[1], mu, rs, wv.y, bv.y),
                                ln_apply(v[2], mu, rs, wv.z, bv.z), ln_apply(v[3], mu, rs, wv.w, bv.w)};
            if constexpr (NT == 1) {
                const int k = 4 * lane;
                *reinterpret_cast<float4*>(&sA[f32_lo(k)][ffn::a_off(r, f32_col(k))]) = make_float4(y[0], y[1], y[2], y[3]);
            } else {
                uint2 hp, lp;
                split4(y[0], y[1], y[2], y[3], hp, lp);
                const int o = ffn::a_off(r, 4 * lane);
                *reinterpret_cast<uint2*>(&sA[0][o]) = hp;
                *reinterpret_cast<uint2*>(&sA[1][o]) = lp;
            }
        }
    }
    __syncthreads();

    const int ar = lane & 15, kq = 8 * (lane >> 4), m_of = 4 * (lane >> 4);
    const __amdgpu_buffer_rsrc_t wip = wbuf(Wip), wxp = wbuf(Wxp);
    // in_proj chunk k (columns CH k .. CH k + 63; chunks 0..7 are x, 8..15 are z): wave w computes columns
    // CH k + 16 w .. + 15 for all 64 rows, with the weight block (fragment 4 k + w, K step s) as the A operand
    // (mfma_split_step_t): lane l holds columns 16 w + m_of + r of row 16 i + ar.  The 8 blocks of a chunk
    // stream through 8 register slots, slot s reloaded with K step s of the next chunk right after its use.
    // Chunk order: z first (8..15), then x (0..7).
    constexpr int R1 = 8, NCH = 2 * DI / CH;
    auto chunk_of = [](int i) { return i < NCH / 2 ? NCH / 2 + i : i - NCH / 2; };  // i-th chunk processed
    u32x4 r1h[R1], r1l[R1];
    auto issue_w = [&](int k, int s) {  // block (fragment 4 k + wave, K step s) into slot s
        const uint32_t bo = (uint32_t)((((CH / 16) * k + wave) * (D / 32) + s) * BLK * 2);
        r1h[s] = wbuf_ld16(wip, lane * 16, bo);
        r1l[s] = r1h[s];
        if constexpr (two_part_blocks<NT>()) r1l[s] = wbuf_ld16(wip, lane * 16, bo + 1024);
    };
#pragma unroll
    for (int s = 0; s < R1; ++s) issue_w(chunk_of(0), s);
    floatx4 dacc[3];  // x_proj (dbc) of rows 16 wave .. + 15, fragments 0..2
#pragma unroll
    for (int j = 0; j < 3; ++j) dacc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int s1 = p0m3 == 2 ? 0 : p0m3 + 1, s2 = p0m3 == 0 ? 2 : p0m3 - 1;

#pragma unroll 1
    for (int ci = 0; ci < NCH; ++ci) {
        const int k = chunk_of(ci);
        const int kn = chunk_of(ci + 1 < NCH ? ci + 1 : ci);
        const int cl0 = 16 * wave + m_of;  // first of this lane's 4 columns within the chunk
        // loaded ahead of the ring's next blocks: its use must not wait for them (in-order wait counter)
        const float4 bias = ldg_f4(G(bin) + CH * k + cl0);
        floatx4 acc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < D / 32; ++s) {
            bf16x8 ah[4], al[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int o = ffn::a_off(16 * i + ar, 32 * s + kq);
                ah[i] = *reinterpret_cast<const bf16x8*>(&sA[0][o]);
                al[i] = *reinterpret_cast<const bf16x8*>(&sA[1][o]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[i] = mfma_split_step_t<NT>(acc[i], ah[i], al[i], __builtin_bit_cast(bf16x8, r1h[s]),
                                               __builtin_bit_cast(bf16x8, r1l[s]));
            issue_w(kn, s);
            pin_loads();
        }
        if (k >= NCH / 2) {
            // z chunk: straight to HBM (the scan reads it)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                stg_f4(GM(xz) + (m0 + 16 * i + ar) * (2 * DI) + CH * k + cl0,
                       make_float4(epi_value<EPI_BIAS>(acc[i][0], bias.x), epi_value<EPI_BIAS>(acc[i][1], bias.y),
                                   epi_value<EPI_BIAS>(acc[i][2], bias.z), epi_value<EPI_BIAS>(acc[i][3], bias.w)));
            continue;
        }
        // x chunk: fp32 to LDS for the conv over time
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<float4*>(&sX[sx_off(16 * i + ar, cl0)]) =
                make_float4(epi_value<EPI_BIAS>(acc[i][0], bias.x), epi_value<EPI_BIAS>(acc[i][1], bias.y),
                            epi_value<EPI_BIAS>(acc[i][2], bias.z), epi_value<EPI_BIAS>(acc[i][3], bias.w));
        __syncthreads();
        // conv + SiLU: thread = (channel cl, rows 16 g .. 16 g + 15); inputs read before the barrier, the split
        // output written over them after it.  g is the wave index, so the history descriptors below are
        // wave-uniform: wave 0 reads the 3 history inputs (the others read nothing: empty range, value 0) and
        // wave 3 writes the ring back; no memory access sits under a branch.
        bf16x8 xwh[2][3], xwl[2][3];  // x_proj weight blocks of K block k (in flight during the conv)
        {
            const int cl = tid & (CH - 1), g = wave;
            const int c = CH * k + cl;
            const float4 cw = ldg_f4(G(conv_w) + 4 * c);
            const float cb = G(conv_b)[c];
            const __amdgpu_buffer_rsrc_t hr =
                buf_rsrc(hist + b * 3 * DI, g == 0 ? 3 * DI * 4 : 0);
            const float h0 = buf_ld1(hr, (uint32_t)(p0m3 * DI + c) * 4), h1 = buf_ld1(hr, (uint32_t)(s1 * DI + c) * 4),
                        h2 = buf_ld1(hr, (uint32_t)(s2 * DI + c) * 4);
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    const uint32_t bo = (uint32_t)((j * (DI / 32) + 2 * k + s) * BLK * 2);
                    const u32x4 bh = wbuf_ld16(wxp, lane * 16, bo);
                    xwh[s][j] = __builtin_bit_cast(bf16x8, bh);
                    xwl[s][j] = two_part_blocks<NT>() ? __builtin_bit_cast(bf16x8, wbuf_ld16(wxp, lane * 16, bo + 1024))
                                                      : xwh[s][j];
                }
            pin_loads();
            float xv[19];
#pragma unroll
            for (int e = 0; e < 3; ++e) xv[e] = sX[sx_off(g == 0 ? 0 : 16 * g - 3 + e, cl)];
#pragma unroll
            for (int e = 0; e < 16; ++e) xv[3 + e] = sX[sx_off(16 * g + e, cl)];
            __syncthreads();
            if (g == 0) {
                xv[0] = h0;
                xv[1] = h1;
                xv[2] = h2;
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int r = 16 * g + e;
                const float y = conv_point(cw, cb, xv[e], xv[e + 1], xv[e + 2], xv[e + 3]);
                GM(xs)[(m0 + r) * DI + c] = y;
                if constexpr (NT == 1) {
                    *reinterpret_cast<float*>((f32_lo(cl) ? sXl : sXh) + x_off(r, f32_col(cl))) = y;
                } else {
                    uint32_t hi, lo;
                    split2(y, hi, lo);
                    sXh[x_off(r, cl)] = (uint16_t)hi;
                    sXl[x_off(r, cl)] = (uint16_t)lo;
                }
            }
            // history ring: inputs of positions p0 + 61, 62, 63 in slots (p0 + 64) mod 3, + 1, + 2 (wave 3)
            const int e0 = (p0m3 + BM) % 3, e1 = (e0 + 1) % 3, e2 = (e0 + 2) % 3;
            const __amdgpu_buffer_rsrc_t hw = buf_rsrc(hist + b * 3 * DI, g == BM / 16 - 1 ? 3 * DI * 4 : 0);
            buf_st1(hw, (uint32_t)(e0 * DI + c) * 4, xv[16]);
            buf_st1(hw, (uint32_t)(e1 * DI + c) * 4, xv[17]);
            buf_st1(hw, (uint32_t)(e2 * DI + c) * 4, xv[18]);
        }
        __syncthreads();
        // x_proj partial over this chunk's 64 channels (K block k, from zero): rows 16 wave .. + 15, fragments
        // 0..2, folded into dbc in ascending block order (XPROJ_KB; every mode)
        {
            floatx4 part[3];
#pragma unroll
            for (int j = 0; j < 3; ++j) part[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const int o = x_off(16 * wave + ar, 32 * s + kq);
                const bf16x8 ah = *reinterpret_cast<const bf16x8*>(&sXh[o]);
                const bf16x8 al = *reinterpret_cast<const bf16x8*>(&sXl[o]);
#pragma unroll
                for (int j = 0; j < 3; ++j) part[j] = mfma_split_step<NT>(part[j], ah, al, xwh[s][j], xwl[s][j]);
            }
#pragma unroll
            for (int j = 0; j < 3; ++j) dacc[j] = k == 0 ? part[j] : dacc[j] + part[j];
        }
        __syncthreads();  // the next x chunk rewrites sX
    }
    // dbc rows 16 wave .. + 15
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) GM(dbc)[(m0 + 16 * wave + m_of + r) * FW + 16 * j + ar] = dacc[j][r];
    // layer 0 of a compress tile: the embedding rows to x (the residual stream), gathered again from the table
    // (an L2 hit) and stored after the tile's other work (stored in the prologue instead: the same time)
    if constexpr (EMB) {
#pragma unroll 4
        for (int q = 0; q < BM / 4; ++q)
            *reinterpret_cast<float4*>(e.xout + (m0 + 16 * wave + q) * D + 4 * lane) =
                ldg_f4(G(e.emb) + (int64_t)__builtin_amdgcn_readlane(tokv, q) * D + 4 * lane);
    }
}

// The mixer's input half for d_model 512 (d_inner 1024, dt_rank 32, x_proj width 64; configs[4]'s shape), one
// lane's tile of 64 positions per workgroup: LN1 -> in_proj (+bias) -> z to HBM; x -> causal conv + SiLU over the
// tile -> xs to HBM -> x_proj, folded over 64-channel K blocks (XPROJ_KB) in registers -> dbc to HBM; the conv
// history ring advanced by 64 positions.  The same arithmetic per value as k_mixin and the layer-by-layer
// kernels.  The LN1 operand is 128 KB, so one workgroup runs per CU, with 8 waves (2 per SIMD):
//   in_proj: per 64-column chunk, wave w computes rows 32 (w & 1) .. + 31 x columns 16 (w >> 1) .. + 15, the
//            weight block as the A operand (each block read by two waves); 16 K steps through a ring of 16
//            register slots (8 with bf16x3 weights, whose blocks are twice the size) running on into the next
//            chunk;
//   conv:    thread = (channel cl, rows 8 g .. 8 g + 7), g = wave: wave 0 reads the 3 history inputs, wave 7
//            writes the ring back (wave-uniform buffer ranges, no access under a branch);
//   x_proj:  wave w owns rows 16 (w & 3) .. + 15 x output fragments 2 (w >> 2), + 1.
namespace mixin5 {
constexpr int BM = 64, D = 512, DI = 1024, CH = 64, FW = 64;
}  // namespace mixin5

template <int NT, bool EMB>
__global__ void __launch_bounds__(512, 2) k_mixin512(const float* __restrict__ x, const float* __restrict__ ln_w,
                                                     const float* __restrict__ ln_b, const uint16_t* __restrict__ Wip,
                                                     const float* __restrict__ bin, const float* __restrict__ conv_w,
                                                     const float* __restrict__ conv_b, const uint16_t* __restrict__ Wxp,
                                                     float* __restrict__ xz, float* __restrict__ xs,
                                                     float* __restrict__ dbc, float* __restrict__ hist, int p0m3,
                                                     EmbedIn e) {
    using namespace mixin5;
    using mixin::sx_off;
    using mixin::x_off;
    constexpr int BLK = (NT == 3) ? 1024 : 512;
    __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * D];  // LN1 output (hi, lo)
    __shared__ __attribute__((aligned(16))) float sX[BM * CH];        // x chunk fp32; then its conv output split
    uint16_t* sXh = reinterpret_cast<uint16_t*>(sX);
    uint16_t* sXl = sXh + BM * CH;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t b = blockIdx.x, m0 = b * BM;
    // ---- LN1: 8 rows per wave (layer 0 of a compress tile: of the embedding rows, which are also written to x at
    //      the end; lane q of a wave reads the token of its row q, handed to every lane by readlane)
    const int tokv = EMB ? byte_token(e.bytes, e.stride, e.lens, b, e.t0 + 8 * wave + (lane & 7), e.V) : 0;
    {
        const float4 w0 = ldg_f4(G(ln_w) + 4 * lane), w1 = ldg_f4(G(ln_w) + 256 + 4 * lane);
        const float4 c0 = ldg_f4(G(ln_b) + 4 * lane), c1 = ldg_f4(G(ln_b) + 256 + 4 * lane);
        const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        const float bv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll 2
        for (int q = 0; q < BM / 8; ++q) {
            const int r = 8 * wave + q;
            float4 u0, u1;
            if constexpr (EMB) {
                const gptr<float> er = G(e.emb) + (int64_t)__builtin_amdgcn_readlane(tokv, q) * D + 4 * lane;
                u0 = ldg_f4(er);
                u1 = ldg_f4(er + 256);
            } else {
                u0 = ldg_f4(G(x) + (m0 + r) * D + 4 * lane);
                u1 = ldg_f4(G(x) + (m0 + r) * D + 256 + 4 * lane);
            }
            const float v[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
            float mu, rs;
            ln_stats_row<2>(v, mu, rs);
            float y[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) y[i] = ln_apply(v[i], mu, rs, wv[i], bv[i]);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint2 hp, lp;
                split4(y[4 * h], y[4 * h + 1], y[4 * h + 2], y[4 * h + 3], hp, lp);
                const int o = ffn5::a_off(r, 256 * h + 4 * lane);
                *reinterpret_cast<uint2*>(&sA[0][o]) = hp;
                *reinterpret_cast<uint2*>(&sA[1][o]) = lp;
            }
        }
    }
    __syncthreads();

    const int ar = lane & 15, kq = 8 * (lane >> 4), m_of = 4 * (lane >> 4);
    const gptr<uint16_t> wip = G(Wip), wxp = G(Wxp);
    const int rh = wave & 1, cf = wave >> 1;
    constexpr int NS1 = D / 32, R1 = NT == 3 ? 8 : NS1, NCH = 2 * DI / CH;  // K steps per chunk, ring slots
    auto chunk_of = [](int i) { return i < NCH / 2 ? NCH / 2 + i : i - NCH / 2; };  // z chunks first, then x
    u32x4 r1h[R1], r1l[R1];
    auto issue_w = [&](int k, int s) {  // block (fragment 4 k + cf, K step s) into slot s % R1
        const gptr<uint16_t> q = wip + ((int64_t)((CH / 16) * k + cf) * (D / 32) + s) * BLK + lane * 8;
        r1h[s % R1] = ldg16(q);
        r1l[s % R1] = r1h[s % R1];
        if constexpr (NT == 3) r1l[s % R1] = ldg16(q + 512);
    };
#pragma unroll
    for (int s = 0; s < R1; ++s) issue_w(chunk_of(0), s);
    const int xr = wave & 3, xf = 2 * (wave >> 2);  // x_proj: row fragment, first output fragment
    floatx4 dacc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) dacc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int s1 = p0m3 == 2 ? 0 : p0m3 + 1, s2 = p0m3 == 0 ? 2 : p0m3 - 1;

#pragma unroll 1
    for (int ci = 0; ci < NCH; ++ci) {
        const int k = chunk_of(ci);
        const int kn = chunk_of(ci + 1 < NCH ? ci + 1 : ci);
        const int cl0 = 16 * cf + m_of;  // first of this lane's 4 columns within the chunk
        const float4 bias = ldg_f4(G(bin) + CH * k + cl0);
        floatx4 acc[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < NS1; ++s) {
            bf16x8 ah[2], al[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int o = ffn5::a_off(32 * rh + 16 * i + ar, 32 * s + kq);
                ah[i] = *reinterpret_cast<const bf16x8*>(&sA[0][o]);
                al[i] = *reinterpret_cast<const bf16x8*>(&sA[1][o]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
                acc[i] = mfma_split_step_t<NT>(acc[i], ah[i], al[i], __builtin_bit_cast(bf16x8, r1h[s % R1]),
                                               __builtin_bit_cast(bf16x8, r1l[s % R1]));
            if (s + R1 < NS1) issue_w(k, s + R1);  // resolved at compile time
            else issue_w(kn, s + R1 - NS1);
            pin_loads();
        }
        if (k >= NCH / 2) {
            // z chunk: straight to HBM (the scan reads it)
#pragma unroll
            for (int i = 0; i < 2; ++i)
                stg_f4(GM(xz) + (m0 + 32 * rh + 16 * i + ar) * (2 * DI) + CH * k + cl0,
                       make_float4(epi_value<EPI_BIAS>(acc[i][0], bias.x), epi_value<EPI_BIAS>(acc[i][1], bias.y),
                                   epi_value<EPI_BIAS>(acc[i][2], bias.z), epi_value<EPI_BIAS>(acc[i][3], bias.w)));
            continue;
        }
        // x chunk: fp32 to LDS for the conv over time
#pragma unroll
        for (int i = 0; i < 2; ++i)
            *reinterpret_cast<float4*>(&sX[sx_off(32 * rh + 16 * i + ar, cl0)]) =
                make_float4(epi_value<EPI_BIAS>(acc[i][0], bias.x), epi_value<EPI_BIAS>(acc[i][1], bias.y),
                            epi_value<EPI_BIAS>(acc[i][2], bias.z), epi_value<EPI_BIAS>(acc[i][3], bias.w));
        __syncthreads();
        bf16x8 xwh[2][2], xwl[2][2];  // x_proj weight blocks of K block k for this wave's two fragments
        {
            const int cl = tid & (CH - 1), g = wave;
            const int c = CH * k + cl;
            const float4 cw = ldg_f4(G(conv_w) + 4 * c);
            const float cb = G(conv_b)[c];
            const __amdgpu_buffer_rsrc_t hr = buf_rsrc(hist + b * 3 * DI, g == 0 ? 3 * DI * 4 : 0);
            const float h0 = buf_ld1(hr, (uint32_t)(p0m3 * DI + c) * 4), h1 = buf_ld1(hr, (uint32_t)(s1 * DI + c) * 4),
                        h2 = buf_ld1(hr, (uint32_t)(s2 * DI + c) * 4);
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const gptr<uint16_t> q = wxp + ((int64_t)(xf + j) * (DI / 32) + 2 * k + s) * BLK + lane * 8;
                    const u32x4 bh = ldg16(q);
                    xwh[s][j] = __builtin_bit_cast(bf16x8, bh);
                    xwl[s][j] = NT == 3 ? __builtin_bit_cast(bf16x8, ldg16(q + 512)) : xwh[s][j];
                }
            pin_loads();
            float xv[11];
#pragma unroll
            for (int e = 0; e < 3; ++e) xv[e] = sX[sx_off(g == 0 ? 0 : 8 * g - 3 + e, cl)];
#pragma unroll
            for (int e = 0; e < 8; ++e) xv[3 + e] = sX[sx_off(8 * g + e, cl)];
            __syncthreads();
            if (g == 0) {
                xv[0] = h0;
                xv[1] = h1;
                xv[2] = h2;
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int r = 8 * g + e;
                const float y = conv_point(cw, cb, xv[e], xv[e + 1], xv[e + 2], xv[e + 3]);
                GM(xs)[(m0 + r) * DI + c] = y;
                uint32_t hi, lo;
                split2(y, hi, lo);
                sXh[x_off(r, cl)] = (uint16_t)hi;
                sXl[x_off(r, cl)] = (uint16_t)lo;
            }
            // history ring: inputs of positions p0 + 61, 62, 63 in slots (p0 + 64) mod 3, + 1, + 2 (wave 7)
            const int e0 = (p0m3 + BM) % 3, e1 = (e0 + 1) % 3, e2 = (e0 + 2) % 3;
            const __amdgpu_buffer_rsrc_t hw = buf_rsrc(hist + b * 3 * DI, g == BM / 8 - 1 ? 3 * DI * 4 : 0);
            buf_st1(hw, (uint32_t)(e0 * DI + c) * 4, xv[8]);
            buf_st1(hw, (uint32_t)(e1 * DI + c) * 4, xv[9]);
            buf_st1(hw, (uint32_t)(e2 * DI + c) * 4, xv[10]);
        }
        __syncthreads();
        // x_proj partial over this chunk's 64 channels (K block k)
        {
            floatx4 part[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) part[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const int o = x_off(16 * xr + ar, 32 * s + kq);
                const bf16x8 ah = *reinterpret_cast<const bf16x8*>(&sXh[o]);
                const bf16x8 al = *reinterpret_cast<const bf16x8*>(&sXl[o]);
#pragma unroll
                for (int j = 0; j < 2; ++j) part[j] = mfma_split_step<NT>(part[j], ah, al, xwh[s][j], xwl[s][j]);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) dacc[j] = k == 0 ? part[j] : dacc[j] + part[j];
        }
        __syncthreads();  // the next x chunk rewrites sX
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) GM(dbc)[(m0 + 16 * xr + m_of + r) * FW + 16 * (xf + j) + ar] = dacc[j][r];
    // layer 0 of a compress tile: the embedding rows to x, gathered again and stored last (as in k_mixin)
    if constexpr (EMB) {
#pragma unroll 2
        for (int q = 0; q < BM / 8; ++q) {
            const gptr<float> er = G(e.emb) + (int64_t)__builtin_amdgcn_readlane(tokv, q) * D + 4 * lane;
            float* xr_ = e.xout + (m0 + 8 * wave + q) * D + 4 * lane;
            *reinterpret_cast<float4*>(xr_) = ldg_f4(er);
            *reinterpret_cast<float4*>(xr_ + 256) = ldg_f4(er + 256);
        }
    }
}

// fp32 mode: the K-block fold over the fp32 weight matrix (k_xproj_f32)
static int launch_xproj_f32(const float* xs, int64_t M, int di, const float* W, float* dbc, int ldd, hipStream_t s) {
    const unsigned grid = (unsigned)((M + 63) / 64);
    if (di % XPROJ_KB != 0) return boa_fail(BOA_ERR_ARG, "internal: d_inner %d not a multiple of %d", di, XPROJ_KB);
    if (ldd == 48) hipLaunchKernelGGL((k_xproj_f32<3>), dim3(grid), dim3(256), 0, s, xs, M, di, W, dbc, ldd);
    else if (ldd == 64) hipLaunchKernelGGL((k_xproj_f32<4>), dim3(grid), dim3(256), 0, s, xs, M, di, W, dbc, ldd);
    else return boa_fail(BOA_ERR_ARG, "internal: x_proj width %d not supported (48 or 64)", ldd);
    return BOA_OK;
}

static int launch_xproj(const float* xs, int64_t M, int di, const uint16_t* Wh, const uint16_t* Wl, float* dbc, int ldd,
                        hipStream_t s) {
    const unsigned grid = (unsigned)((M + 63) / 64);
    if (di % XPROJ_KB != 0) return boa_fail(BOA_ERR_ARG, "internal: d_inner %d not a multiple of %d", di, XPROJ_KB);
    if (ldd == 48) {
        if (Wl) hipLaunchKernelGGL((k_xproj<3, 3>), dim3(grid), dim3(256), 0, s, xs, M, di, Wh, Wl, dbc, ldd);
        else hipLaunchKernelGGL((k_xproj<2, 3>), dim3(grid), dim3(256), 0, s, xs, M, di, Wh, Wl, dbc, ldd);
    } else if (ldd == 64) {
        if (Wl) hipLaunchKernelGGL((k_xproj<3, 4>), dim3(grid), dim3(256), 0, s, xs, M, di, Wh, Wl, dbc, ldd);
        else hipLaunchKernelGGL((k_xproj<2, 4>), dim3(grid), dim3(256), 0, s, xs, M, di, Wh, Wl, dbc, ldd);
    } else {
        return boa_fail(BOA_ERR_ARG, "internal: x_proj width %d not supported (48 or 64)", ldd);
    }
    return BOA_OK;
}

// ================================================================================================
// Selective scan, fused with dt_proj + softplus, the D skip and the SiLU(z) gate (the Mamba mixer's step,
// reference portability_solved_cpp/mamba_kernels.cu:264-347 and its chunked form :396-444):
//   dt = softplus(W_dt . dr + b_dt)                  (torch threshold 20)
//   h_n <- exp(dt * A_n) * h_n + B_n * (dt * x)      A = -exp(A_log), precomputed as A * log2(e) so the
//                                                    16 exponentials per position are exp2 (v_exp_f32)
//   y = sum_n h_n * C_n + D * x ;  y <- y * SiLU(z)
// One thread per (lane, channel), h[16] in registers across the Tc positions.  The [dr | B | C] row of a
// position is uniform across the workgroup and read-only here, so the compiler reads it with scalar loads
// into SGPRs (3 x 16 dwords per position): no LDS staging, no per-position LDS reads, and 76 VGPRs at
// d_model 256 with fp32 output, which gives 6 waves per SIMD instead of 5 (the scan is latency-bound at that
// occupancy: 346 -> 316 ms per 16 MiB).  x and z of the next two positions are in flight while one computes
// (a three-slot register ring), and the state update writes each h_n over its own register (scan_update's
// INPLACE form).  State [lane][di][NS] in HBM between launches.  y overwrites x in place.
// The per-position arithmetic is scan_position (shared with the fused decompress-step kernel).

template <int NS, int R>
__device__ __forceinline__ void scan_load_channel(int c, int di, const float* hp, const float* Aneg, const float* dt_w,
                                                  float (&h)[NS], float (&a)[NS], float (&wr)[R]) {
#pragma unroll
    for (int n = 0; n < NS; n += 4) {
        const float4 q = *reinterpret_cast<const float4*>(hp + (int64_t)(n / 4) * di * 4);
        h[n] = q.x; h[n + 1] = q.y; h[n + 2] = q.z; h[n + 3] = q.w;
        const float4 p = *reinterpret_cast<const float4*>(Aneg + ((int64_t)(n / 4) * di + c) * 4);
        a[n] = p.x; a[n + 1] = p.y; a[n + 2] = p.z; a[n + 3] = p.w;
    }
#pragma unroll
    for (int r = 0; r < R; r += 4) {
        const float4 q = *reinterpret_cast<const float4*>(dt_w + (int64_t)c * R + r);
        wr[r] = q.x; wr[r + 1] = q.y; wr[r + 2] = q.z; wr[r + 3] = q.w;
    }
}

template <int NS>
__device__ __forceinline__ void scan_store_channel(float* hp, int di, const float (&h)[NS]) {
#pragma unroll
    for (int n = 0; n < NS; n += 4)
        *reinterpret_cast<float4*>(hp + (int64_t)(n / 4) * di * 4) = make_float4(h[n], h[n + 1], h[n + 2], h[n + 3]);
}

// Output of one position: fp32 in place of x (fp32 GEMM mode) or split bf16 parts (split modes).
template <bool OUTS>
__device__ __forceinline__ void scan_store_y(float* xs_y, uint16_t* yh, uint16_t* yl, int64_t idx, float y) {
    if constexpr (OUTS) {
        uint32_t h, l;
        split2(y, h, l);
        yh[idx] = (uint16_t)h;
        yl[idx] = (uint16_t)l;
    } else {
        xs_y[idx] = y;
    }
}

// Tile kernel (compress path): Tc positions per lane, h in registers across them.
template <int NS, int R, bool OUTS>
__global__ void __launch_bounds__(256) k_scan(float* __restrict__ xs_y, const float* __restrict__ dbc, int ldd,
                                             const float* __restrict__ xz, int64_t ldxz,
                                             const float* __restrict__ dt_w, const float* __restrict__ dt_b,
                                             const float* __restrict__ Aneg, const float* __restrict__ Dp,
                                             float* __restrict__ ssm, int di, int Tc, uint16_t* __restrict__ yh,
                                             uint16_t* __restrict__ yl) {
    const int64_t b = blockIdx.y;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t row0 = b * Tc;
    if (c >= di) return;
    float h[NS], a[NS], wr[R];
    float* hp = ssm + b * di * NS + 4 * c;
    scan_load_channel<NS, R>(c, di, hp, Aneg, dt_w, h, a, wr);
    const float bdt = dt_b[c], Dc = Dp[c];
    // x and z of positions t + 1 and t + 2 in flight while position t computes: a ring of three register slots,
    // position t in slot t % 3 (the loop unrolled by three), reloaded with position t + 3 once used; loads past
    // the tile repeat its last position (read before that position's y is written over it, and unused)
    float xr[3], zr[3];
    auto ld = [&](int t, int u) {
        const int64_t m = row0 + (t < Tc ? t : Tc - 1);
        xr[u] = xs_y[m * di + c];
        zr[u] = xz[m * ldxz + di + c];
    };
    ld(0, 0);
    ld(1, 1);
    for (int t0 = 0; t0 < Tc; t0 += 3) {
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            const int t = t0 + u;
            if (t < Tc) {
                ld(t + 2, (u + 2) % 3);
                const int64_t m = row0 + t;
                scan_store_y<OUTS>(xs_y, yh, yl, m * di + c,
                                   scan_position<NS, R, true>(dbc + m * ldd, wr, bdt, a, Dc, xr[u], zr[u], h));
            }
        }
    }
    scan_store_channel<NS>(hp, di, h);
}

// Step kernel (decompress path, per-layer kernels): one position per lane.  A workgroup owns 256 channels of
// SCAN_LPB consecutive lanes: each channel's parameters (A, its dt_proj row, biases) are loaded once for all of
// them, and each lane's 64 B of state per channel stream through range-checked non-temporal buffer accesses
// (lanes past B read 0 and are not written, so no state access is under a branch), the next lane's state
// loaded before the current lane computes.  The [dr | B | C] row of a lane is uniform across the workgroup.
constexpr int SCAN_LPB = 8;
template <int NS, int R, bool OUTS>
__global__ void __launch_bounds__(256) k_scan_step(float* __restrict__ xs_y, const float* __restrict__ dbc, int ldd,
                                                  const float* __restrict__ xz, int64_t ldxz,
                                                  const float* __restrict__ dt_w, const float* __restrict__ dt_b,
                                                  const float* __restrict__ Aneg, const float* __restrict__ Dp,
                                                  float* __restrict__ ssm, int di, int B, uint16_t* __restrict__ yh,
                                                  uint16_t* __restrict__ yl) {
    const int c = blockIdx.x * 256 + threadIdx.x;  // di is a multiple of 256
    const int64_t b0 = (int64_t)blockIdx.y * SCAN_LPB;
    const int nb = (int)((B - b0) < SCAN_LPB ? (B - b0) : SCAN_LPB);
    float a[NS], wr[R];
#pragma unroll
    for (int n = 0; n < NS; n += 4) {
        const float4 p = ldg_f4(G(Aneg) + ((int64_t)(n / 4) * di + c) * 4);
        a[n] = p.x; a[n + 1] = p.y; a[n + 2] = p.z; a[n + 3] = p.w;
    }
#pragma unroll
    for (int r = 0; r < R; r += 4) {
        const float4 q = ldg_f4(G(dt_w) + (int64_t)c * R + r);
        wr[r] = q.x; wr[r + 1] = q.y; wr[r + 2] = q.z; wr[r + 3] = q.w;
    }
    const float bdt = G(dt_b)[c], Dc = G(Dp)[c];
    const __amdgpu_buffer_rsrc_t sr = buf_rsrc(ssm + b0 * di * NS, (uint32_t)nb * di * NS * 4);
    auto h_off = [&](int r, int n) { return (uint32_t)(((int64_t)r * NS / 4 + n / 4) * di + c) * 16; };
    f32x4 nxt[NS / 4];
#pragma unroll
    for (int n = 0; n < NS; n += 4) nxt[n / 4] = buf_ld4(sr, h_off(0, n));
#pragma unroll
    for (int r = 0; r < SCAN_LPB; ++r) {
        float h[NS];
#pragma unroll
        for (int n = 0; n < NS; n += 4) {
            h[n] = nxt[n / 4].x; h[n + 1] = nxt[n / 4].y; h[n + 2] = nxt[n / 4].z; h[n + 3] = nxt[n / 4].w;
        }
        if (r + 1 < SCAN_LPB) {  // resolved at compile time
#pragma unroll
            for (int n = 0; n < NS; n += 4) nxt[n / 4] = buf_ld4(sr, h_off(r + 1, n));
        }
        const int64_t b = b0 + (r < nb ? r : nb - 1);  // rows past B repeat the last lane's inputs, unused
        const float x = xs_y[b * di + c];
        const float z = xz[b * ldxz + di + c];
        const float y = scan_position<NS, R>(dbc + b * ldd, wr, bdt, a, Dc, x, z, h);
        if (r < nb) scan_store_y<OUTS>(xs_y, yh, yl, b * di + c, y);
#pragma unroll
        for (int n = 0; n < NS; n += 4) buf_st4(sr, h_off(r, n), f32x4{h[n], h[n + 1], h[n + 2], h[n + 3]});
    }
}

// ================================================================================================
// Fused coder kernels (quantiser XQ at PRECISION 24), one wavefront per chunk lane.
__global__ void k_enc_init(EncState* st, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) enc_init(st[i]);
}

// cumulative of symbol s and its weight, from the owner lane (s uniform across the wave)
__device__ __forceinline__ void xq_sym(const XQ& q, int s, uint32_t& c_s, uint32_t& f_s) {
    const int j = s & 3;
    uint32_t cl = q.base, fl = q.f[0];
    if (j >= 1) { cl += q.f[0]; fl = q.f[1]; }
    if (j >= 2) { cl += q.f[1]; fl = q.f[2]; }
    if (j >= 3) { cl += q.f[2]; fl = q.f[3]; }
    c_s = wave_bcast(cl, s >> 2);
    f_s = wave_bcast(fl, s >> 2);
}

// Encodes the symbols predicted by the Tc positions of this launch: the logits of position p (absolute
// t0 + t) code byte p + 1 of the chunk (codec.py:56-76: step(byte t-1) -> probabilities of byte t).
__global__ void __launch_bounds__(64) k_encode_tile(const float* __restrict__ logits, int V, int Tc, int t0,
                                                   const uint8_t* __restrict__ bytes, int64_t stride,
                                                   const int32_t* __restrict__ lens, EncState* __restrict__ states,
                                                   uint32_t* __restrict__ words, int64_t pitch) {
    const int64_t b = blockIdx.x;
    const int lane = threadIdx.x;
    const int L = lens[b];
    if (t0 + 1 >= L) return;
    EncState st = states[b];
    const WordSink sink{words + b * pitch, pitch, lane == 0};
    const uint8_t* src = bytes + b * stride;
    for (int t = 0; t < Tc; ++t) {
        const int p = t0 + t;
        if (p + 1 >= L) break;
        const int s = src[p + 1];
        if (s >= V) continue;  // as gpu_range_coder.py:97: symbols outside [0, K) are skipped
        XQ q;
        xq_build(q, logits_row4(logits + (b * Tc + t) * V, V, lane), lane, V, CODER_P);
        uint32_t c_s, f_s;
        xq_sym(q, s, c_s, f_s);
        const uint32_t lo = xq_cdf_at(q, c_s, s);
        const uint32_t hi = (s + 1 < V) ? xq_cdf_at(q, c_s + f_s, s + 1) : (1u << CODER_P);
        enc_push(st, CODER_P, lo, hi - lo, sink);
    }
    if (lane == 0) states[b] = st;
}

// ================================================================================================
// Head + quantiser of a compress tile, fused: for the Tc = 64 positions of one chunk lane,
//   logits = W2 . ReLU(W1 . x + b1) + b2            (model.py:95,101: Linear -> ReLU -> Linear)
// then the fused quantiser (XQ) of each position's logits row and the coder interval [lo, lo + width) of the
// byte that position predicts (codec.py:56-76: step(byte t-1) -> probabilities of byte t), written as one
// (lo, width) pair per position for k_encode_lf, which runs the sequential range coder.  The reference does
// head, quantised table and encode per time step from logits in HBM (range_coder_kernels.cu:612-748,
// ker_rc_encode_chunk_parallel_warp); here the logits never leave the chip.
// The arithmetic of every value is that of the tiled head GEMMs and of the fused decode kernel: x split by
// split4; head1 outputs accumulate their D/32 K steps in ascending order (mfma_split_step_t: the same value as
// mfma_split_step), then epi_value<RELU>, split; head2 outputs accumulate all D/32 K steps in ascending order
// (64-unit chunks of the hidden layer, in order), then epi_value<BIAS>.  The logits, and so the tables, equal
// the decoder's bit for bit.
// 512 threads (8 waves).  Per 64-unit chunk c of the hidden layer: head1 wave tile 32 rows x 16 units (the W1
// block as the A operand, a lane's 4 outputs are consecutive units: one 8-byte store per part), then head2
// accumulates the chunk: wave w owns logits 32 w .. + 31 (2 fragments) of all 64 rows.  A wave's weight blocks
// (D/32 of W1, then 4 of W2 per chunk) stream through one 4-slot register ring in use order, as in k_ffn.
// LDS: x operand [64][D] (hi, lo) + hidden chunk [64][64] (hi, lo); the logits [64][260] fp32 reuse it.
// D = 256: 80 KB, two workgroups per CU; D = 512: 144 KB, one.
namespace headq {
constexpr int BM = 64, V = 256, HC = 64, LLOG = V + 4;
constexpr uint32_t SKIP = 0xFFFFFFFFu;  // no symbol at this position (past the chunk's end, or byte >= V)
// 16-byte chunks XOR-swizzled by row (low 4 bits of the chunk index), so 16-row fragment reads spread over banks
template <int D> __device__ __forceinline__ int a_off(int r, int k) { return r * D + (((k >> 3) ^ (r & 15)) << 3) + (k & 7); }
__device__ __forceinline__ int h_off(int r, int k) { return r * HC + (((k >> 3) ^ (r >> 1)) & 7) * 8 + (k & 7); }
template <int D> constexpr int lds_bytes() {
    return (2 * BM * D * 2 + 2 * BM * HC * 2) > BM * LLOG * 4 ? (2 * BM * D * 2 + 2 * BM * HC * 2) : BM * LLOG * 4;
}
}  // namespace headq

template <int NT, int D>
__global__ void __launch_bounds__(512, (D == 256) ? 4 : 2) k_head_xq(const float* __restrict__ xin,
                                                                   const uint16_t* __restrict__ W1p,
                                                                   const float* __restrict__ b1,
                                                                   const uint16_t* __restrict__ W2p,
                                                                   const float* __restrict__ b2, int t0,
                                                                   const uint8_t* __restrict__ bytes, int64_t stride,
                                                                   const int32_t* __restrict__ lens,
                                                                   uint2* __restrict__ lf) {
    using namespace headq;
    __shared__ __attribute__((aligned(16))) unsigned char lds[lds_bytes<D>()];
    uint16_t* sAh = reinterpret_cast<uint16_t*>(lds);
    uint16_t* sAl = sAh + BM * D;
    uint16_t* sHh = sAl + BM * D;
    uint16_t* sHl = sHh + BM * HC;
    float* sLog = reinterpret_cast<float*>(lds);  // after the last chunk
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t b = blockIdx.x;
    {
        const gptr<float> xr = G(xin) + b * BM * D;
#pragma unroll 4
        for (int q = 0; q < BM / 8; ++q) {
            const int r = 8 * wave + q;
#pragma unroll
            for (int h = 0; h < D / 256; ++h) {
                const float4 v = ldg_f4(xr + r * D + 256 * h + 4 * lane);
                if constexpr (NT == 1) {
                    const int k = 256 * h + 4 * lane;
                    *reinterpret_cast<float4*>((f32_lo(k) ? sAl : sAh) + a_off<D>(r, f32_col(k))) = v;
                } else {
                    uint2 hp, lp;
                    split4(v.x, v.y, v.z, v.w, hp, lp);
                    const int o = a_off<D>(r, 256 * h + 4 * lane);
                    *reinterpret_cast<uint2*>(sAh + o) = hp;
                    *reinterpret_cast<uint2*>(sAl + o) = lp;
                }
            }
        }
    }
    const int ar = lane & 15, m_of = 4 * (lane >> 4);
    __syncthreads();
    constexpr int BLK = two_part_blocks<NT>() ? 1024 : 512;
    const __amdgpu_buffer_rsrc_t w1p = wbuf(W1p), w2p = wbuf(W2p);
    const int rh = wave & 1, cf = wave >> 1;
    constexpr int KS = D / 32, NBC = KS + 4, R = 4, NC = D / HC;
    static_assert(NBC % R == 0 && KS % R == 0, "ring slots divide the blocks of a chunk");
    u32x4 rhh[R], rll[R];
    auto issue = [&](int c, int i) {
        const int blk = i < KS ? (4 * c + cf) * KS + i : (2 * wave + ((i - KS) & 1)) * KS + 2 * c + ((i - KS) >> 1);
        const __amdgpu_buffer_rsrc_t wr = i < KS ? w1p : w2p;
        rhh[i % R] = wbuf_ld16(wr, lane * 16, (uint32_t)(blk * BLK * 2));
        rll[i % R] = rhh[i % R];
        if constexpr (two_part_blocks<NT>()) rll[i % R] = wbuf_ld16(wr, lane * 16, (uint32_t)(blk * BLK * 2 + 1024));
    };
    auto refill = [&](int c, int cn, int i) {
        if (i + R < NBC) issue(c, i + R);
        else issue(cn, i + R - NBC);
    };
    floatx4 out[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) out[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < R; ++i) issue(0, i);
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
        const int cn = c + 1 < NC ? c + 1 : c;
        const float4 bias = ldg_f4(G(b1) + HC * c + 16 * cf + m_of);
        floatx4 hacc[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) hacc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
        // LDS addresses are formed per chunk from an opaque copy of the lane index: hoisted out of the chunk
        // loop they would hold a dozen registers, which spill (and every reload waits behind the weight ring)
        int lq = lane;
        __asm__ volatile("" : "+v"(lq));
        const int arq = lq & 15, kqq = 8 * (lq >> 4);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            bf16x8 ah[2], al[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int o = a_off<D>(32 * rh + 16 * i + arq, 32 * s + kqq);
                ah[i] = *reinterpret_cast<const bf16x8*>(sAh + o);
                al[i] = *reinterpret_cast<const bf16x8*>(sAl + o);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
                hacc[i] = mfma_split_step_t<NT>(hacc[i], ah[i], al[i], __builtin_bit_cast(bf16x8, rhh[s % R]),
                                                __builtin_bit_cast(bf16x8, rll[s % R]));
            refill(c, cn, s);
            pin_loads();
        }
        {
            const float bv[4] = {bias.x, bias.y, bias.z, bias.w};
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                float g[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) g[r] = epi_value<EPI_RELU>(hacc[i][r], bv[r]);
                if constexpr (NT == 1) {
                    const int k = 16 * cf + m_of;
                    *reinterpret_cast<float4*>((f32_lo(k) ? sHl : sHh) + h_off(32 * rh + 16 * i + ar, f32_col(k))) =
                        make_float4(g[0], g[1], g[2], g[3]);
                } else {
                    uint2 hp, lp;
                    split4(g[0], g[1], g[2], g[3], hp, lp);
                    const int o = h_off(32 * rh + 16 * i + ar, 16 * cf + m_of);
                    *reinterpret_cast<uint2*>(sHh + o) = hp;
                    *reinterpret_cast<uint2*>(sHl + o) = lp;
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            bf16x8 ah[4], al[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int o = h_off(16 * i + arq, 32 * t + kqq);
                ah[i] = *reinterpret_cast<const bf16x8*>(sHh + o);
                al[i] = *reinterpret_cast<const bf16x8*>(sHl + o);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int bi = KS + 2 * t + j;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    out[i][j] = mfma_split_step<NT>(out[i][j], ah[i], al[i], __builtin_bit_cast(bf16x8, rhh[bi % R]),
                                                    __builtin_bit_cast(bf16x8, rll[bi % R]));
                refill(c, cn, bi);
                pin_loads();
            }
        }
        __syncthreads();
    }
    // the operand and hidden buffers are dead (the last chunk ended with a barrier): logits in their place
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int col = 16 * (2 * wave + j) + ar;
        const float bias = G(b2)[col];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) sLog[(16 * i + m_of + r) * LLOG + col] = epi_value<EPI_BIAS>(out[i][j][r], bias);
    }
    __syncthreads();
    // quantiser and coder interval per position: wave w takes positions 8 w .. 8 w + 7 (uniform per wave)
    const int L = lens[b];
    const uint8_t* src = bytes + b * stride;
#pragma unroll 1
    for (int q = 0; q < BM / 8; ++q) {
        const int t = 8 * wave + q;
        const int p = t0 + t;
        uint2 v = make_uint2(SKIP, 0u);
        if (p + 1 < L) {
            const int s = src[p + 1];
            if (s < V) {
                XQ xq;
                xq_build(xq, logits_row4(sLog + t * LLOG, V, lane), lane, V, CODER_P);
                uint32_t c_s, f_s;
                xq_sym(xq, s, c_s, f_s);
                const uint32_t lo = xq_cdf_at(xq, c_s, s);
                const uint32_t hi = (s + 1 < V) ? xq_cdf_at(xq, c_s + f_s, s + 1) : (1u << CODER_P);
                v = make_uint2(lo, hi - lo);
            }
        }
        if (lane == 0) lf[b * BM + t] = v;
    }
}

// The sequential coder over one tile's (lo, width) pairs (k_head_xq), one thread per chunk lane.
__global__ void __launch_bounds__(256) k_encode_lf(const uint2* __restrict__ lf, int Tc, int n,
                                                  EncState* __restrict__ states, uint32_t* __restrict__ words,
                                                  int64_t pitch) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n) return;
    EncState st = states[b];
    const WordSink sink{words + b * pitch, pitch, true};
    const uint2* q = lf + b * Tc;
    for (int t = 0; t < Tc; ++t) {
        const uint2 v = q[t];
        if (v.x == headq::SKIP) continue;
        enc_push(st, CODER_P, v.x, v.y, sink);
    }
    states[b] = st;
}

__global__ void k_enc_finish(EncState* states, uint32_t* words, int64_t pitch, int32_t* nwords, int32_t* overflow,
                             int n) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n) return;
    EncState st = states[b];
    const WordSink sink{words + (int64_t)b * pitch, pitch, true};
    enc_finish(st, sink);
    states[b] = st;
    nwords[b] = st.overflow ? 0 : st.nwords;
    if (st.overflow) overflow[0] = 1;
}

__global__ void k_dec_init(DecState* states, const uint32_t* payload, int64_t payload_words, const int64_t* off,
                           const int32_t* nwords, const uint8_t* first, const int32_t* lens, int32_t* tokens,
                           uint8_t* out, int64_t out_stride, int n) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n) return;
    DecState st;
    const LaneWords w = lane_words(payload, payload_words, off, nwords, b);
    dec_init(st, w.p, w.n);
    states[b] = st;
    tokens[b] = first[b];
    if (lens[b] >= 1) out[(int64_t)b * out_stride] = first[b];
}

// One decode step at position t for every lane with t < len: quantise the logits, find the symbol the
// coder state points into, advance the state, emit the byte and feed it back as the next token.
__global__ void __launch_bounds__(64) k_decode_step(const float* __restrict__ logits, int V, int t,
                                                   const int32_t* __restrict__ lens, DecState* __restrict__ states,
                                                   const uint32_t* __restrict__ payload, int64_t payload_words,
                                                   const int64_t* __restrict__ off, const int32_t* __restrict__ nwords,
                                                   int32_t* __restrict__ tokens, uint8_t* __restrict__ out,
                                                   int64_t out_stride) {
    const int64_t b = blockIdx.x;
    const int lane = threadIdx.x;
    if (t >= lens[b]) return;
    DecState st = states[b];
    const LaneWords w = lane_words(payload, payload_words, off, nwords, b);
    const int s = decode_row(logits + b * V, V, lane, st, w.p, w.n);
    if (lane == 0) {
        states[b] = st;
        tokens[b] = s;
        out[b * out_stride + t] = (uint8_t)s;
    }
}

// Scatter of a tile's logits [B*Tc][V] into [B][len][V] at positions t0..t0+Tc-1.
__global__ void __launch_bounds__(256) k_scatter_logits(const float* __restrict__ src, int V, int Tc, int t0,
                                                       int len, int64_t rows, float* __restrict__ dst) {
    const int64_t m = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (m >= rows) return;
    const int64_t b = m / Tc;
    const int t = (int)(m - b * Tc);
    const float* s = src + m * V;
    float* d = dst + (b * len + t0 + t) * V;
    for (int c = lane; c < V; c += 64) d[c] = s[c];
}

// ================================================================================================
// Context

// A GEMM weight matrix [N][K]: fp32 values plus, in the split-precision modes, bf16 parts (hi, lo).
struct MatW {
    const float* f = nullptr;
    const uint16_t* h = nullptr;
    const uint16_t* l = nullptr;
    const uint16_t* p = nullptr;  // fragment-packed parts (fused step kernel)
    int64_t n = 0;
    int N = 0, K = 0;
};

struct LayerW {
    const float *ln1_w, *ln1_b, *in_b, *conv_w, *conv_b, *dt_w, *dt_b, *A_log, *D, *out_b, *ln2_w, *ln2_b, *ff1_b,
        *ff2_b;
    MatW in_w, x_w, out_w, ff1_w, ff2_w;
    float* Aneg;
};

static GemmArgs gemm_args(const float* A, int64_t lda, const MatW& W, const float* bias, float* C, int64_t ldc,
                          int64_t M, int N, int K) {
    GemmArgs g;
    memset(&g, 0, sizeof(g));
    g.A = A; g.lda = lda; g.W = W.f; g.Wh = W.h; g.Wl = W.l; g.bias = bias; g.C = C; g.ldc = ldc;
    g.M = M; g.N = N; g.K = K;
    return g;
}

// Per-kernel-class event timing (boa_profile / boa_profile_read).
enum ProfClass {
    PC_EMBED, PC_IN, PC_CONV, PC_XPROJ, PC_SCAN, PC_OUT, PC_FF1, PC_FF2, PC_HEAD1, PC_HEAD2, PC_ENCODE, PC_DECODE,
    PC_LN, PC_FUSED, PC_FFN, PC_MIXIN, PC_HEADXQ, PC_COUNT
};
static const char* kProfNames[PC_COUNT] = {"embed",    "gemm_in_proj", "conv",     "gemm_x_proj",
                                           "scan",     "gemm_out_proj", "gemm_ff1", "gemm_ff2",
                                           "gemm_head1", "gemm_head2", "encode",   "decode",
                                           "ln_stats", "fused_step", "ffn", "mixin", "head_xq"};
struct ProfClassState {
    int64_t launches = 0;
    int64_t used = 0;
    double flops = 0.0, bytes = 0.0;
    std::vector<hipEvent_t> ev;  // 2 per sampled launch, created on first use and reused
};

struct boa_ctx {
    boa_model_cfg cfg;
    int d, di, NS, R, V, L, DC;
    hipStream_t stream = nullptr;
    int32_t max_lanes = 0, tile_len = 0;
    int64_t max_rows = 0;
    float* wblob = nullptr;
    float* aneg = nullptr;
    const float *emb = nullptr, *h1_b = nullptr, *h2_b = nullptr;
    MatW h1_w, h2_w;
    int prec = BOA_PREC_F32;
    uint16_t* wsplit = nullptr;
    std::vector<LayerW> layers;
    float* conv_hist = nullptr;  // [L][max_lanes][3][di]
    float* ssm = nullptr;        // [L][max_lanes][NS/4][di][4]
    float *x = nullptr, *xz = nullptr, *xs = nullptr, *dbc = nullptr, *mm = nullptr, *logits = nullptr;
    float2* stats = nullptr;
    uint16_t *ah = nullptr, *al = nullptr;  // split activations [max_rows][max(d, di)] (split modes)
    int32_t* tokens = nullptr;
    EncState* enc = nullptr;
    DecState* dec = nullptr;
    int32_t* flag = nullptr;
    int64_t pos = 0;                   // positions processed since the last state reset (conv history ring)
    bool fused = false;                // decompress / step through k_fused_step
    int fused_steps = 128;             // decode steps per k_fused_step launch
    // k_fused_step workgroup classes (sets of XCDs) can start this far apart, so that one class runs its
    // HBM-bound scans while the other streams weights from L2.  Off by default: with the recurrent state
    // streamed non-temporally the weights stay in L2 and offsets of 0-450 us measure the same.
    int stagger_us = 0;
    int stagger_classes = 2;
    // Per-layer decode in two halves of the lanes on two streams (contexts without the fused decode kernel):
    // one half's state-bound groups (conv + scan) run while the other half's GEMM groups run.  lane0 shifts
    // the per-lane state of the launches (0 outside the second half).
    int decode_halves = 2;
    bool ffn_outp = true;  // out_proj inside the feed-forward kernel (BOA_FFN_OUTP=0: separate GEMM)
    bool head_xq = true;   // compress tiles: head + quantiser in one kernel (BOA_HEAD_XQ=0: head GEMMs + k_encode_tile)
    // full compress tiles: layer 0's mixer-input kernel gathers the embedding rows itself instead of the separate
    // embedding pass (BOA_EMBED_LN1=0: the pass).  emb_src is the current tile's (set only around its layer-0
    // launch).
    bool embed_ln1 = true;
    EmbedIn emb_src;
    // compress in groups of the lanes on their own streams (BOA_COMPRESS_HALVES=0: one stream; BOA_COMPRESS_GROUPS:
    // 2 or 3 groups, default 2)
    bool compress_halves = true;
    int compress_groups = 2;
    hipStream_t stream2 = nullptr;
    hipStream_t stream3 = nullptr;     // the third compress group's
    std::vector<hipEvent_t> half_ev;   // [2][L]: state group of layer l done, per half; [2L], [2L + 1]: stream joins
    int64_t lane0 = 0;
    uint16_t* wfrag = nullptr;         // fragment-packed GEMM weights (fused)
    FusedLayer* d_layers = nullptr;    // per-layer pointer table (fused)
    int64_t device_bytes = 0;
    bool prof_on = false;
    ProfClassState prof[PC_COUNT];
};

// Returns the event-pair index of this launch, or -1 when not sampled.
static int64_t prof_start(boa_ctx* x, int cls) {
    if (!x->prof_on) return -1;
    ProfClassState& p = x->prof[cls];
    if (p.used >= BOA_PROF_SAMPLES) return -1;
    const int64_t i = p.used;
    if ((int64_t)p.ev.size() < 2 * (i + 1)) {
        hipEvent_t a, b;
        if (hipEventCreate(&a) != hipSuccess) return -1;
        if (hipEventCreate(&b) != hipSuccess) { (void)hipEventDestroy(a); return -1; }
        p.ev.push_back(a);
        p.ev.push_back(b);
    }
    if (hipEventRecord(p.ev[2 * i], x->stream) != hipSuccess) return -1;
    return i;
}

static void prof_stop(boa_ctx* x, int cls, int64_t i, double flops, double bytes) {
    if (!x->prof_on) return;
    ProfClassState& p = x->prof[cls];
    p.launches++;
    if (i < 0) return;
    if (hipEventRecord(p.ev[2 * i + 1], x->stream) != hipSuccess) return;
    p.used = i + 1;
    p.flops += flops;
    p.bytes += bytes;
}

extern "C" int boa_profile(boa_ctx* x, int enable) {
    if (!x) return boa_fail(BOA_ERR_ARG, "boa_profile: null context");
    if (enable) {
        for (auto& p : x->prof) { p.launches = 0; p.used = 0; p.flops = 0.0; p.bytes = 0.0; }
    }
    x->prof_on = enable != 0;
    return BOA_OK;
}

extern "C" int boa_profile_read(boa_ctx* x, boa_prof_entry* out, int32_t cap, int32_t* n) {
    if (!x || !n || (cap > 0 && !out)) return boa_fail(BOA_ERR_ARG, "boa_profile_read: bad arguments");
    BOA_HIP_TRY(hipStreamSynchronize(x->stream));
    int32_t k = 0;
    for (int c = 0; c < PC_COUNT; ++c) {
        const ProfClassState& p = x->prof[c];
        if (p.launches == 0) continue;
        if (k < cap) {
            boa_prof_entry& e = out[k];
            memset(&e, 0, sizeof(e));
            snprintf(e.name, sizeof(e.name), "%s", kProfNames[c]);
            e.launches = p.launches;
            e.sampled = p.used;
            double ms = 0.0;
            for (int64_t i = 0; i < p.used; ++i) {
                float t = 0.0f;
                BOA_HIP_TRY(hipEventElapsedTime(&t, p.ev[2 * i], p.ev[2 * i + 1]));
                ms += t;
            }
            e.ms = ms;
            e.flops = p.flops;
            e.bytes = p.bytes;
        }
        ++k;
    }
    *n = k;
    return BOA_OK;
}

static int64_t weights_floats(const boa_model_cfg& c, int R) {
    const int64_t d = c.d_model, di = (int64_t)c.expand * c.d_model, NS = c.d_state, V = c.vocab, DC = c.d_conv;
    const int64_t per = 2 * d + 2 * di * d + 2 * di + di * DC + di + (R + 2 * NS) * di + di * R + di + di * NS + di +
                        d * di + d + 2 * d + 4 * d * d + 4 * d + d * 4 * d + d;
    return V * d + c.n_layers * per + d * d + d + V * d + V;
}

static int resolve_cfg(const boa_model_cfg* in, boa_model_cfg& c, int& R) {
    if (!in) return boa_fail(BOA_ERR_ARG, "null model config");
    c = *in;
    if (c.d_state == 0) c.d_state = 16;
    if (c.d_conv == 0) c.d_conv = 4;
    if (c.expand == 0) c.expand = 2;
    R = c.dt_rank > 0 ? c.dt_rank : (c.d_model + 15) / 16;
    c.dt_rank = R;
    if (c.d_model != 256 && c.d_model != 512)
        return boa_fail(BOA_ERR_ARG, "d_model must be 256 or 512 (got %d)", c.d_model);
    if (c.n_layers < 1 || c.n_layers > 64) return boa_fail(BOA_ERR_ARG, "n_layers out of range (%d)", c.n_layers);
    if (c.vocab < 2 || c.vocab > 256) return boa_fail(BOA_ERR_ARG, "vocab must be in [2, 256] (got %d)", c.vocab);
    if (c.d_state != 16) return boa_fail(BOA_ERR_ARG, "d_state must be 16 (got %d)", c.d_state);
    if (c.d_conv != 4) return boa_fail(BOA_ERR_ARG, "d_conv must be 4 (got %d)", c.d_conv);
    if (c.expand != 2) return boa_fail(BOA_ERR_ARG, "expand must be 2 (got %d)", c.expand);
    if (R != 16 && R != 32) return boa_fail(BOA_ERR_ARG, "dt_rank must be 16 or 32 (got %d)", R);
    if (c.vocab % 4 != 0) return boa_fail(BOA_ERR_ARG, "vocab must be a multiple of 4 (got %d)", c.vocab);
    return BOA_OK;
}

extern "C" int64_t boa_weights_nbytes(const boa_model_cfg* cfg) {
    boa_model_cfg c;
    int R;
    if (resolve_cfg(cfg, c, R) != BOA_OK) return -1;
    return weights_floats(c, R) * 4;
}

extern "C" int64_t boa_ctx_device_bytes(const boa_ctx* ctx) { return ctx ? ctx->device_bytes : 0; }

// Whether a context of this shape and precision decodes through a fused step kernel (BOA_FUSED_STEP=0 turns it
// off): k_fused_step at d_model 256 in every precision mode, k_fused_step512 at d_model 512 in the split modes.
// Whether an fp32-mode context gets fp32 fragment-packed weights: at d_model 256 (the fused decode kernel and
// the fused compress kernels k_mixin, k_ffn, k_head_xq read them), whether or not BOA_FUSED_STEP turns the
// fused decode off.
static bool f32_packed(const boa_model_cfg& c, int R, int precision) {
    return precision == BOA_PREC_F32 && fused_step_supported(c.d_model, c.d_state, R, c.d_conv, c.vocab);
}

static bool want_fused(const boa_model_cfg& c, int R, int precision) {
    const char* fenv = getenv("BOA_FUSED_STEP");
    const bool d256 = fused_step_supported(c.d_model, c.d_state, R, c.d_conv, c.vocab);
    const bool d512 = fused_step512_supported(c.d_model, c.d_state, R, c.d_conv, c.vocab);
    return (d256 || (d512 && precision != BOA_PREC_F32)) && !(fenv && fenv[0] == '0');
}

// Device bytes boa_ctx_create allocates for this shape: the same list of buffers, in the same order, each
// rounded as dmalloc rounds it.  boa_ctx_create checks its own total against this after allocating.
static int64_t ctx_plan_bytes(const boa_model_cfg& c, int R, int precision, int64_t max_lanes, int64_t tile_len) {
    const int64_t d = c.d_model, di = (int64_t)c.expand * c.d_model, NS = c.d_state, V = c.vocab, L = c.n_layers;
    const int64_t rows = max_lanes * tile_len;
    auto f4 = [](int64_t n) { return 4 * std::max<int64_t>(n, 1); };
    int64_t b = f4(weights_floats(c, R)) + f4(L * di * NS) + f4(L * max_lanes * 3 * di) + f4(L * max_lanes * di * NS) +
                f4(rows * d) + f4(rows * std::max(2 * di, 4 * d)) + f4(rows * di) + f4(rows * (R + 2 * NS)) +
                f4(rows * d) + f4(rows * V) + 8 * std::max<int64_t>(rows, 1);
    if (precision != BOA_PREC_F32) b += 2 * 2 * std::max<int64_t>(rows * std::max(d, di), 1);
    b += f4(max_lanes) + (int64_t)sizeof(EncState) * max_lanes + (int64_t)sizeof(DecState) * max_lanes + 4;
    const int64_t mats = L * (2 * di * d + (R + 2 * NS) * di + d * di + 4 * d * d + 4 * d * d) + d * d + V * d;
    if (precision != BOA_PREC_F32) {
        b += 2 * std::max<int64_t>(2 * mats, 1);
        b += 2 * std::max<int64_t>((precision == BOA_PREC_BF16X3 ? 2 : 1) * mats, 1);
    } else if (f32_packed(c, R, precision)) {
        b += 2 * std::max<int64_t>(2 * mats, 1);  // fp32 fragment-packed weights, in 16-bit units
    }
    if (want_fused(c, R, precision)) b += (int64_t)sizeof(FusedLayer) * L;
    return b;
}

extern "C" int boa_ctx_plan_bytes(const boa_model_cfg* cfg, int precision, int32_t max_lanes, int32_t tile_len,
                                  int64_t* out_bytes) {
    boa_model_cfg c;
    int R;
    if (!out_bytes) return boa_fail(BOA_ERR_ARG, "boa_ctx_plan_bytes: null output");
    int rc = resolve_cfg(cfg, c, R);
    if (rc != BOA_OK) return rc;
    if (max_lanes < 1 || tile_len < 1 || tile_len > 256)
        return boa_fail(BOA_ERR_ARG, "need max_lanes >= 1 and 1 <= tile_len <= 256 (got %d, %d)", max_lanes, tile_len);
    *out_bytes = ctx_plan_bytes(c, R, precision, max_lanes, tile_len);
    return BOA_OK;
}

extern "C" int boa_ctx_destroy(boa_ctx* ctx) {
    if (!ctx) return BOA_OK;
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    else (void)hipDeviceSynchronize();
    void* ptrs[] = {ctx->wblob, ctx->aneg, ctx->conv_hist, ctx->ssm, ctx->x, ctx->xz, ctx->xs, ctx->dbc,
                    ctx->mm, ctx->logits, ctx->stats, ctx->tokens, ctx->enc, ctx->dec, ctx->flag, ctx->wsplit,
                    ctx->ah, ctx->al, ctx->wfrag, ctx->d_layers};
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
    for (auto& p : ctx->prof)
        for (hipEvent_t e : p.ev) (void)hipEventDestroy(e);
    for (hipEvent_t e : ctx->half_ev) (void)hipEventDestroy(e);
    if (ctx->stream2) (void)hipStreamDestroy(ctx->stream2);
    if (ctx->stream3) (void)hipStreamDestroy(ctx->stream3);
    delete ctx;
    return BOA_OK;
}

template <typename T>
static hipError_t dmalloc(boa_ctx* c, T** p, int64_t count) {
    const int64_t bytes = std::max<int64_t>(count, 1) * (int64_t)sizeof(T);
    c->device_bytes += bytes;
    return hipMalloc((void**)p, (size_t)bytes);
}

// Host-side round to nearest even of a float to bfloat16 bits (finite inputs).
static uint16_t host_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static float host_bf16_to_f(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

// The fp32 fragment order of the fused decode kernel's fp32 mode: blocks (f, g) for f < N/16, g < K/16, f-major;
// lane l of a block holds W[16 f + l % 16][16 g + 4 (l / 16) + j], j < 4 (one 16-byte load per lane).
static void pack_fragments_f32(const float* w, int N, int K, float* out) {
    const int S = K / 16;
    for (int f = 0; f < N / 16; ++f)
        for (int g = 0; g < S; ++g) {
            float* o = out + ((int64_t)f * S + g) * 256;
            for (int l = 0; l < 64; ++l)
                for (int j = 0; j < 4; ++j)
                    o[l * 4 + j] = w[(int64_t)(16 * f + (l & 15)) * K + 16 * g + 4 * (l >> 4) + j];
        }
}

// Fragment order for the fused kernel's B operands (layout in model_internal.h).
static void pack_fragments(const uint16_t* hi, const uint16_t* lo, int N, int K, bool two, uint16_t* out) {
    const int S = K / 32, blk = two ? 1024 : 512;
    for (int f = 0; f < N / 16; ++f)
        for (int s = 0; s < S; ++s) {
            uint16_t* o = out + ((int64_t)f * S + s) * blk;
            for (int l = 0; l < 64; ++l)
                for (int j = 0; j < 8; ++j) {
                    const int64_t src = (int64_t)(16 * f + (l & 15)) * K + 32 * s + 8 * (l >> 4) + j;
                    o[l * 8 + j] = hi[src];
                    if (two) o[512 + l * 8 + j] = lo[src];
                }
        }
}

extern "C" int boa_ctx_create(const boa_model_cfg* cfg, const void* h_weights, int64_t nbytes, int precision,
                              int32_t max_lanes, int32_t tile_len, void* stream, boa_ctx** out) {
    if (!out) return boa_fail(BOA_ERR_ARG, "boa_ctx_create: null output");
    *out = nullptr;
    boa_model_cfg c;
    int R;
    int rc = resolve_cfg(cfg, c, R);
    if (rc != BOA_OK) return rc;
    if (precision != BOA_PREC_F32 && precision != BOA_PREC_BF16X3 && precision != BOA_PREC_BF16W)
        return boa_fail(BOA_ERR_ARG, "boa_ctx_create: unknown precision mode %d", precision);
    const int64_t nf = weights_floats(c, R);
    if (!h_weights || nbytes != nf * 4)
        return boa_fail(BOA_ERR_ARG, "weight blob must be %lld bytes (got %lld)", (long long)(nf * 4), (long long)nbytes);
    if (max_lanes < 1 || tile_len < 1 || tile_len > 256)
        return boa_fail(BOA_ERR_ARG, "need max_lanes >= 1 and 1 <= tile_len <= 256 (got %d, %d)", max_lanes, tile_len);
    const int64_t max_rows = (int64_t)max_lanes * tile_len;
    if (max_rows > (int64_t)1 << 31) return boa_fail(BOA_ERR_ARG, "max_lanes * tile_len too large");

    boa_ctx* x = new boa_ctx();
    x->cfg = c;
    x->d = c.d_model; x->di = c.expand * c.d_model; x->NS = c.d_state; x->R = R; x->V = c.vocab;
    x->L = c.n_layers; x->DC = c.d_conv;
    x->stream = reinterpret_cast<hipStream_t>(stream);
    x->prec = precision;
    x->max_lanes = max_lanes; x->tile_len = tile_len; x->max_rows = max_rows;
    const int d = x->d, di = x->di, NS = x->NS, V = x->V, L = x->L;

    hipError_t e = hipSuccess;
#define TRY_ALLOC(p, n) do { if (e == hipSuccess) e = dmalloc(x, &(p), (n)); } while (0)
    TRY_ALLOC(x->wblob, nf);
    TRY_ALLOC(x->aneg, (int64_t)L * di * NS);
    TRY_ALLOC(x->conv_hist, (int64_t)L * max_lanes * 3 * di);
    TRY_ALLOC(x->ssm, (int64_t)L * max_lanes * di * NS);
    TRY_ALLOC(x->x, max_rows * d);
    TRY_ALLOC(x->xz, max_rows * std::max(2 * di, 4 * d));
    TRY_ALLOC(x->xs, max_rows * di);
    TRY_ALLOC(x->dbc, max_rows * (R + 2 * NS));
    TRY_ALLOC(x->mm, max_rows * d);
    TRY_ALLOC(x->logits, max_rows * V);
    TRY_ALLOC(x->stats, max_rows);
    if (precision != BOA_PREC_F32) {
        TRY_ALLOC(x->ah, max_rows * std::max(d, di));
        TRY_ALLOC(x->al, max_rows * std::max(d, di));
    }
    TRY_ALLOC(x->tokens, (int64_t)max_lanes);
    TRY_ALLOC(x->enc, (int64_t)max_lanes);
    TRY_ALLOC(x->dec, (int64_t)max_lanes);
    TRY_ALLOC(x->flag, 1);
#undef TRY_ALLOC
    if (e != hipSuccess) {
        boa_ctx_destroy(x);
        return boa_fail_hip(e, "boa_ctx_create allocation", __FILE__, __LINE__);
    }
    // weight pointers in the flat blob (convert_boa_weights.py:22-133 order)
    const float* hw = static_cast<const float*>(h_weights);
    int64_t o = 0;
    auto take = [&](int64_t n) { const float* p = x->wblob + o; o += n; return p; };
    x->emb = take((int64_t)V * d);
    std::vector<float> aneg_host((size_t)L * di * NS);
    auto mat = [&](int N, int K) {
        MatW m;
        m.n = (int64_t)N * K;
        m.f = take(m.n);
        m.N = N;
        m.K = K;
        return m;
    };
    for (int l = 0; l < L; ++l) {
        LayerW w;
        w.ln1_w = take(d); w.ln1_b = take(d);
        w.in_w = mat(2 * di, d); w.in_b = take(2 * di);
        w.conv_w = take((int64_t)di * x->DC); w.conv_b = take(di);
        w.x_w = mat(R + 2 * NS, di);
        w.dt_w = take((int64_t)di * R); w.dt_b = take(di);
        const int64_t a_off = o;
        w.A_log = take((int64_t)di * NS);
        w.D = take(di);
        w.out_w = mat(d, di); w.out_b = take(d);
        w.ln2_w = take(d); w.ln2_b = take(d);
        w.ff1_w = mat(4 * d, d); w.ff1_b = take(4 * d);
        w.ff2_w = mat(d, 4 * d); w.ff2_b = take(d);
        w.Aneg = x->aneg + (int64_t)l * di * NS;
        // A = -exp(A_log), stored pre-scaled by log2(e) so that exp(dt * A) = exp2(dt * A2); layout [NS/4][di][4]
        for (int64_t c = 0; c < di; ++c)
            for (int n = 0; n < NS; ++n)
                aneg_host[(size_t)l * di * NS + ((size_t)(n / 4) * di + c) * 4 + (n % 4)] =
                    (float)(-exp((double)hw[a_off + c * NS + n]) * 1.4426950408889634);
        x->layers.push_back(w);
    }
    x->h1_w = mat(d, d); x->h1_b = take(d);
    x->h2_w = mat(V, d); x->h2_b = take(V);
    if (o != nf) {
        boa_ctx_destroy(x);
        return boa_fail(BOA_ERR_ARG, "internal: weight layout mismatch (%lld vs %lld)", (long long)o, (long long)nf);
    }
    // GEMM weight copies for the MFMA kernels.  Split-precision modes: bf16 parts of every matrix ([hi | lo] per
    // matrix) and their fragment-packed form, read by the fused compress kernels (k_mixin, k_ffn, k_ffn512,
    // k_head_xq) and the fused decode kernels.  fp32 mode at d_model 256: the fp32 fragment-packed form, read by
    // the same kernels' fp32 forms.
    std::vector<uint16_t> split_host, frag_host;
    std::vector<float> frag32_host;
    std::vector<FusedLayer> layers_host;
    std::vector<MatW*> mats;
    for (auto& w : x->layers) { mats.push_back(&w.in_w); mats.push_back(&w.x_w); mats.push_back(&w.out_w);
                                mats.push_back(&w.ff1_w); mats.push_back(&w.ff2_w); }
    mats.push_back(&x->h1_w);
    mats.push_back(&x->h2_w);
    x->fused = want_fused(c, R, x->prec);
    if (const char* v = getenv("BOA_FUSED_STEPS_PER_LAUNCH")) x->fused_steps = std::max(1, atoi(v));
    if (const char* v = getenv("BOA_FUSED_STAGGER_US")) x->stagger_us = std::max(0, atoi(v));
    if (const char* v = getenv("BOA_FUSED_STAGGER_CLASSES")) x->stagger_classes = std::min(8, std::max(1, atoi(v)));
    if (x->prec != BOA_PREC_F32) {
        int64_t total = 0;
        for (MatW* m : mats) total += 2 * m->n;
        if (e == hipSuccess) e = dmalloc(x, &x->wsplit, total);
        if (e != hipSuccess) {
            boa_ctx_destroy(x);
            return boa_fail_hip(e, "boa_ctx_create allocation", __FILE__, __LINE__);
        }
        split_host.resize((size_t)total);
        int64_t so = 0;
        for (MatW* m : mats) {
            const float* src = hw + (m->f - x->wblob);
            uint16_t* hi = split_host.data() + so;
            uint16_t* lo = hi + m->n;
            for (int64_t i = 0; i < m->n; ++i) {
                hi[i] = host_bf16(src[i]);
                lo[i] = (x->prec == BOA_PREC_BF16X3) ? host_bf16(src[i] - host_bf16_to_f(hi[i])) : (uint16_t)0;
            }
            m->h = x->wsplit + so;
            m->l = (x->prec == BOA_PREC_BF16X3) ? x->wsplit + so + m->n : nullptr;
            so += 2 * m->n;
        }
        const bool two = x->prec == BOA_PREC_BF16X3;
        int64_t ftotal = 0;
        for (MatW* m : mats) ftotal += (two ? 2 : 1) * m->n;
        frag_host.resize((size_t)ftotal);
        if (e == hipSuccess) e = dmalloc(x, &x->wfrag, ftotal);
        int64_t fo = 0, hs = 0;
        for (MatW* m : mats) {
            const uint16_t* hi = split_host.data() + hs;
            pack_fragments(hi, hi + m->n, m->N, m->K, two, frag_host.data() + fo);
            m->p = x->wfrag + fo;
            fo += (two ? 2 : 1) * m->n;
            hs += 2 * m->n;
        }
    } else if (f32_packed(c, R, x->prec)) {
        int64_t ftotal = 0;
        for (MatW* m : mats) ftotal += m->n;
        frag32_host.resize((size_t)ftotal);
        if (e == hipSuccess) e = dmalloc(x, &x->wfrag, 2 * ftotal);  // 16-bit units
        int64_t fo = 0;
        for (MatW* m : mats) {
            pack_fragments_f32(hw + (m->f - x->wblob), m->N, m->K, frag32_host.data() + fo);
            m->p = x->wfrag + 2 * fo;  // fp32 data; the kernel reads it as such
            fo += m->n;
        }
    }
    if (e == hipSuccess && x->fused) e = dmalloc(x, &x->d_layers, (int64_t)L);
    if (e != hipSuccess) {
        boa_ctx_destroy(x);
        return boa_fail_hip(e, "boa_ctx_create allocation", __FILE__, __LINE__);
    }
    if (x->fused) layers_host.resize((size_t)L);
    for (int l = 0; l < (x->fused ? L : 0); ++l) {
        const LayerW& w = x->layers[l];
        FusedLayer& f = layers_host[(size_t)l];
        f.ln1_w = w.ln1_w; f.ln1_b = w.ln1_b; f.in_b = w.in_b; f.conv_w = w.conv_w; f.conv_b = w.conv_b;
        f.dt_w = w.dt_w; f.dt_b = w.dt_b; f.Aneg = w.Aneg; f.D = w.D; f.out_b = w.out_b;
        f.ln2_w = w.ln2_w; f.ln2_b = w.ln2_b; f.ff1_b = w.ff1_b; f.ff2_b = w.ff2_b;
        f.in_p = w.in_w.p; f.x_p = w.x_w.p; f.out_p = w.out_w.p; f.ff1_p = w.ff1_w.p; f.ff2_p = w.ff2_w.p;
    }
    e = hipMemcpyAsync(x->wblob, h_weights, (size_t)nbytes, hipMemcpyHostToDevice, x->stream);
    if (e == hipSuccess && !split_host.empty())
        e = hipMemcpyAsync(x->wsplit, split_host.data(), split_host.size() * 2, hipMemcpyHostToDevice, x->stream);
    if (e == hipSuccess && !frag_host.empty())
        e = hipMemcpyAsync(x->wfrag, frag_host.data(), frag_host.size() * 2, hipMemcpyHostToDevice, x->stream);
    if (e == hipSuccess && !frag32_host.empty())
        e = hipMemcpyAsync(x->wfrag, frag32_host.data(), frag32_host.size() * 4, hipMemcpyHostToDevice, x->stream);
    if (e == hipSuccess && !layers_host.empty())
        e = hipMemcpyAsync(x->d_layers, layers_host.data(), layers_host.size() * sizeof(FusedLayer),
                           hipMemcpyHostToDevice, x->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(x->aneg, aneg_host.data(), aneg_host.size() * 4, hipMemcpyHostToDevice, x->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(x->stream);
    if (e != hipSuccess) {
        boa_ctx_destroy(x);
        return boa_fail_hip(e, "boa_ctx_create upload", __FILE__, __LINE__);
    }
    if (const char* v = getenv("BOA_DECODE_HALVES")) x->decode_halves = atoi(v) == 1 ? 1 : 2;
    if (const char* v = getenv("BOA_FFN_OUTP")) x->ffn_outp = atoi(v) != 0;
    if (const char* v = getenv("BOA_HEAD_XQ")) x->head_xq = atoi(v) != 0;
    if (const char* v = getenv("BOA_EMBED_LN1")) x->embed_ln1 = atoi(v) != 0;
    if (const char* v = getenv("BOA_COMPRESS_HALVES")) x->compress_halves = atoi(v) != 0;
    if (const char* v = getenv("BOA_COMPRESS_GROUPS")) x->compress_groups = atoi(v) == 3 ? 3 : 2;
    if ((!x->fused && x->decode_halves == 2) || x->compress_halves) {
        // default priority (as the context's own stream): streams of different priorities are not mixed
        e = hipStreamCreateWithFlags(&x->stream2, hipStreamNonBlocking);
        if (e == hipSuccess && x->compress_halves && x->compress_groups == 3)
            e = hipStreamCreateWithFlags(&x->stream3, hipStreamNonBlocking);
        for (int i = 0; e == hipSuccess && i < 2 * L + 2; ++i) {
            hipEvent_t ev;
            e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
            if (e == hipSuccess) x->half_ev.push_back(ev);
        }
        if (e != hipSuccess) {
            boa_ctx_destroy(x);
            return boa_fail_hip(e, "boa_ctx_create streams", __FILE__, __LINE__);
        }
    }
    if (x->device_bytes != ctx_plan_bytes(c, R, precision, max_lanes, tile_len)) {
        const long long got = (long long)x->device_bytes, plan = (long long)ctx_plan_bytes(c, R, precision, max_lanes, tile_len);
        boa_ctx_destroy(x);
        return boa_fail(BOA_ERR_STATE, "internal: context holds %lld bytes, plan says %lld", got, plan);
    }
    *out = x;
    return BOA_OK;
}

extern "C" int boa_state_reset(boa_ctx* x, int32_t lanes) {
    if (!x || lanes < 0 || lanes > x->max_lanes) return boa_fail(BOA_ERR_ARG, "boa_state_reset: bad lanes");
    x->pos = 0;
    for (int l = 0; l < x->L; ++l) {
        BOA_HIP_TRY(hipMemsetAsync(x->conv_hist + (int64_t)l * x->max_lanes * 3 * x->di, 0,
                                   sizeof(float) * (size_t)lanes * 3 * x->di, x->stream));
        BOA_HIP_TRY(hipMemsetAsync(x->ssm + (int64_t)l * x->max_lanes * x->di * x->NS, 0,
                                   sizeof(float) * (size_t)lanes * x->di * x->NS, x->stream));
    }
    return BOA_OK;
}

// Launch wrappers that record per-class timing when profiling is on.
#define PROF(cls, flops, bytes, ...)                                \
    do {                                                            \
        const int64_t _pi = prof_start(x, (cls));                   \
        __VA_ARGS__;                                                \
        prof_stop(x, (cls), _pi, (double)(flops), (double)(bytes)); \
    } while (0)

static double gemm_flops(int64_t M, int N, int K) { return 2.0 * (double)M * N * K; }
static double gemm_bytes(int64_t M, int N, int K) { return 4.0 * ((double)M * K + (double)N * K + (double)M * N); }

static void launch_ln_stats(boa_ctx* x, const float* A, int64_t lda, int64_t M) {
    const unsigned blocks = (unsigned)((M + 3) / 4);
    if (x->d == 256)
        PROF(PC_LN, 0.0, 4.0 * M * x->d + 8.0 * M,
             hipLaunchKernelGGL((k_ln_stats<1>), dim3(blocks), dim3(256), 0, x->stream, A, lda, M, x->stats));
    else
        PROF(PC_LN, 0.0, 4.0 * M * x->d + 8.0 * M,
             hipLaunchKernelGGL((k_ln_stats<2>), dim3(blocks), dim3(256), 0, x->stream, A, lda, M, x->stats));
}

// LayerNorm + split into ctx->ah / ctx->al (row stride d).
static void launch_ln_split(boa_ctx* x, const float* A, int64_t M, const float* w, const float* b) {
    const unsigned blocks = (unsigned)((M + 3) / 4);
    const int64_t d = x->d;
    if (x->d == 256)
        PROF(PC_LN, 0.0, 8.0 * M * d,
             hipLaunchKernelGGL((k_ln_split<1>), dim3(blocks), dim3(256), 0, x->stream, A, d, M, w, b, x->ah, x->al));
    else
        PROF(PC_LN, 0.0, 8.0 * M * d,
             hipLaunchKernelGGL((k_ln_split<2>), dim3(blocks), dim3(256), 0, x->stream, A, d, M, w, b, x->ah, x->al));
}

template <int NS, int R, bool OUTS>
static void launch_scan(boa_ctx* x, const LayerW& w, float* ssm, int B, int Tc) {
    const int di = x->di;
    const dim3 grid((di + 255) / 256, B);
    if (Tc == 1)
        hipLaunchKernelGGL((k_scan_step<NS, R, OUTS>), dim3(di / 256, (B + SCAN_LPB - 1) / SCAN_LPB), dim3(256), 0,
                           x->stream, x->xs, x->dbc, R + 2 * NS, x->xz, (int64_t)2 * di, w.dt_w, w.dt_b, w.Aneg, w.D,
                           ssm, di, B, x->ah, x->al);
    else
        hipLaunchKernelGGL((k_scan<NS, R, OUTS>), grid, dim3(256), 0, x->stream, x->xs, x->dbc, R + 2 * NS, x->xz,
                           (int64_t)2 * di, w.dt_w, w.dt_b, w.Aneg, w.D, ssm, di, Tc, x->ah, x->al);
}

// Whether a layer of a Tc-position tile runs LN1 through x_proj as one mixer-input kernel: k_mixin512 (d_model
// 512, split modes) or k_mixin (d_model 256, every mode), on full tiles with fragment-packed weights.
static bool mixin512_layer(const boa_ctx* x, const LayerW& w, int Tc) {
    return x->prec != BOA_PREC_F32 && x->d == mixin5::D && x->di == mixin5::DI && x->R + 2 * x->NS == mixin5::FW &&
           Tc == mixin5::BM && w.in_w.p && w.x_w.p;
}
static bool mixin_layer(const boa_ctx* x, const LayerW& w, int Tc) {
    return !mixin512_layer(x, w, Tc) && x->d == mixin::D && x->di == mixin::DI && x->R + 2 * x->NS == mixin::FW &&
           Tc == mixin::BM && w.in_w.p && w.x_w.p;
}
// Whether a compress tile of Tc positions skips the embedding pass: its layer 0 gathers the rows (EmbedIn).
static bool embed_in_mixin(const boa_ctx* x, int Tc) {
    return x->embed_ln1 && x->L > 0 && (mixin512_layer(x, x->layers[0], Tc) || mixin_layer(x, x->layers[0], Tc));
}

// Sets the context's embedding source for one layer-0 launch sequence of a compress tile and clears it after.
struct EmbedFromBytes {
    boa_ctx* x;
    EmbedFromBytes(boa_ctx* c, bool on, const uint8_t* bytes, int64_t stride, const int32_t* lens, int t0) : x(c) {
        x->emb_src = EmbedIn{};
        if (on) {
            x->emb_src.bytes = bytes; x->emb_src.stride = stride; x->emb_src.lens = lens;
            x->emb_src.emb = x->emb; x->emb_src.t0 = t0; x->emb_src.V = x->V;  // xout: the launch's x
        }
    }
    ~EmbedFromBytes() { x->emb_src = EmbedIn{}; }
};

// One block of the model over B lanes x Tc positions, in place on ctx->x.
//   fp32 mode:  LN stats -> in_proj(LN on load) -> conv -> x_proj -> scan (y in place of xs) -> out_proj ->
//               LN stats -> FF1(LN on load, GELU) into xz -> FF2(+residual) into x
//   split modes: LN+split -> in_proj -> conv -> x_proj -> scan (y split) -> out_proj -> LN+split ->
//               FF1(GELU, split output into xz's memory) -> FF2(+residual) into x
// part selects which of three consecutive groups of the layer to launch (bits, 7 = the whole layer):
//   1: LN1 + in_proj;  2: conv + x_proj + scan (the state traffic);  4: out_proj + LN2 + feed-forward.
// Where a fused compress-tile kernel (k_mixin, k_mixin512) covers LN1 through x_proj, bit 1 launches it and
// bit 2 the scan alone.
static int run_layer(boa_ctx* x, int l, int B, int Tc, int part = 7) {
    const LayerW& w = x->layers[l];
    const int d = x->d, di = x->di, NS = x->NS, R = x->R;
    const int64_t M = (int64_t)B * Tc;
    hipStream_t s = x->stream;
    const bool split = x->prec != BOA_PREC_F32;
    // layer 0 of a tile whose embedding pass was skipped: the mixer-input kernel gathers the rows
    EmbedIn ein = (l == 0) ? x->emb_src : EmbedIn{};
    ein.xout = x->x;
    const bool emb = ein.bytes != nullptr;
    if (emb && !((mixin512_layer(x, w, Tc) || mixin_layer(x, w, Tc)) && (part & 1)))
        return boa_fail(BOA_ERR_STATE, "run_layer: no embedding pass for a tile without the mixer-input kernel");
    // FF hidden activations (split): two bf16 arrays in the memory of xz (dead after the scan)
    uint16_t* gh = reinterpret_cast<uint16_t*>(x->xz);
    uint16_t* gl = gh + M * 4 * d;
    int rc = 0;
    float* hist = x->conv_hist + ((int64_t)l * x->max_lanes + x->lane0) * 3 * di;
    const bool mix5 = mixin512_layer(x, w, Tc);
    if (mix5 && (part & 1)) {
        // LN1 + in_proj + conv + SiLU + x_proj in one kernel per lane tile, d_model 512
        const double flops = gemm_flops(M, 2 * di, d) + gemm_flops(M, R + 2 * NS, di) + 8.0 * M * di;
        const double bytes = 4.0 * M * (d + di + di + R + 2 * NS) + 4.0 * 6 * B * di;
        if (w.in_w.l)
            PROF(PC_MIXIN, flops, bytes,
                 if (emb) hipLaunchKernelGGL((k_mixin512<3, true>), dim3((unsigned)B), dim3(512), 0, s, x->x, w.ln1_w,
                                           w.ln1_b, w.in_w.p, w.in_b, w.conv_w, w.conv_b, w.x_w.p, x->xz, x->xs,
                                           x->dbc, hist, (int)(x->pos % 3), ein);
                 else hipLaunchKernelGGL((k_mixin512<3, false>), dim3((unsigned)B), dim3(512), 0, s, x->x, w.ln1_w,
                                           w.ln1_b, w.in_w.p, w.in_b, w.conv_w, w.conv_b, w.x_w.p, x->xz, x->xs,
                                           x->dbc, hist, (int)(x->pos % 3), ein));
        else
            PROF(PC_MIXIN, flops, bytes,
                 if (emb) hipLaunchKernelGGL((k_mixin512<2, true>), dim3((unsigned)B), dim3(512), 0, s, x->x, w.ln1_w,
                                           w.ln1_b, w.in_w.p, w.in_b, w.conv_w, w.conv_b, w.x_w.p, x->xz, x->xs,
                                           x->dbc, hist, (int)(x->pos % 3), ein);
                 else hipLaunchKernelGGL((k_mixin512<2, false>), dim3((unsigned)B), dim3(512), 0, s, x->x, w.ln1_w,
                                           w.ln1_b, w.in_w.p, w.in_b, w.conv_w, w.conv_b, w.x_w.p, x->xz, x->xs,
                                           x->dbc, hist, (int)(x->pos % 3), ein));
    }
    // (fp32 mode included: its fragment-packed weights exist at d_model 256)
    const bool mix = mixin_layer(x, w, Tc);
    if (mix && (part & 1)) {
        // LN1 + in_proj + conv + SiLU + x_proj in one kernel per lane tile
        const double flops = gemm_flops(M, 2 * di, d) + gemm_flops(M, R + 2 * NS, di) + 8.0 * M * di;
        const double bytes = 4.0 * M * (d + di + di + R + 2 * NS) + 4.0 * 6 * B * di;
        if (x->prec == BOA_PREC_F32)
            PROF(PC_MIXIN, flops, bytes,
                 if (emb) hipLaunchKernelGGL((k_mixin<1, true>), dim3((unsigned)B), dim3(256), 0, s, x->x, w.ln1_w,
                                           w.ln1_b, w.in_w.p, w.in_b, w.conv_w, w.conv_b, w.x_w.p, x->xz, x->xs,
                                           x->dbc, hist, (int)(x->pos % 3), ein);
                 else hipLaunchKernelGGL((k_mixin<1, false>), dim3((unsigned)B), dim3(256), 0, s, x->x, w.ln1_w,
                                           w.ln1_b, w.in_w.p, w.in_b, w.conv_w, w.conv_b, w.x_w.p, x->xz, x->xs,
                                           x->dbc, hist, (int)(x->pos % 3), ein));
        else if (w.in_w.l)
            PROF(PC_MIXIN, flops, bytes,
                 if (emb) hipLaunchKernelGGL((k_mixin<3, true>), dim3((unsigned)B), dim3(256), 0, s, x->x, w.ln1_w,
                                           w.ln1_b, w.in_w.p, w.in_b, w.conv_w, w.conv_b, w.x_w.p, x->xz, x->xs,
                                           x->dbc, hist, (int)(x->pos % 3), ein);
                 else hipLaunchKernelGGL((k_mixin<3, false>), dim3((unsigned)B), dim3(256), 0, s, x->x, w.ln1_w,
                                           w.ln1_b, w.in_w.p, w.in_b, w.conv_w, w.conv_b, w.x_w.p, x->xz, x->xs,
                                           x->dbc, hist, (int)(x->pos % 3), ein));
        else
            PROF(PC_MIXIN, flops, bytes,
                 if (emb) hipLaunchKernelGGL((k_mixin<2, true>), dim3((unsigned)B), dim3(256), 0, s, x->x, w.ln1_w,
                                           w.ln1_b, w.in_w.p, w.in_b, w.conv_w, w.conv_b, w.x_w.p, x->xz, x->xs,
                                           x->dbc, hist, (int)(x->pos % 3), ein);
                 else hipLaunchKernelGGL((k_mixin<2, false>), dim3((unsigned)B), dim3(256), 0, s, x->x, w.ln1_w,
                                           w.ln1_b, w.in_w.p, w.in_b, w.conv_w, w.conv_b, w.x_w.p, x->xz, x->xs,
                                           x->dbc, hist, (int)(x->pos % 3), ein));
    } else if (!mix5 && !mix) {
    // LN1 + in_proj -> xz [M][2di]
    if (part & 1) {
        GemmArgs g = gemm_args(x->x, d, w.in_w, w.in_b, x->xz, 2 * di, M, 2 * di, d);
        if (split) {
            launch_ln_split(x, x->x, M, w.ln1_w, w.ln1_b);
            g.Ah = x->ah; g.Al = x->al;
            PROF(PC_IN, gemm_flops(M, 2 * di, d), gemm_bytes(M, 2 * di, d),
                 rc = (launch_gemm_bf<EPI_BIAS, true, false>(g, s)));
        } else {
            launch_ln_stats(x, x->x, d, M);
            g.ln_w = w.ln1_w; g.ln_b = w.ln1_b; g.ln_stats = x->stats;
            PROF(PC_IN, gemm_flops(M, 2 * di, d), gemm_bytes(M, 2 * di, d),
                 rc = (d == 256) ? launch_gemm_f32<1, EPI_BIAS>(g, s) : launch_gemm_f32<2, EPI_BIAS>(g, s));
        }
        if (rc) return rc;
    }
    if (!(part & 2)) {
        // group 2 not requested
    } else if (split && Tc == 1) {
        // decompress step: conv + SiLU + x_proj in one kernel (same arithmetic as the two kernels below)
        const size_t lds = sizeof(float) * 16 * (size_t)(di + 4);
        const double flops = 8.0 * M * di + gemm_flops(M, R + 2 * NS, di);
        const double bytes = 4.0 * (3.0 * M * di + 6.0 * B * di + M * (R + 2 * NS));
        if (w.x_w.l)
            PROF(PC_CONV, flops, bytes,
                 hipLaunchKernelGGL((k_convx_step<3>), dim3((B + 15) / 16), dim3(256), lds, s, x->xz, (int64_t)2 * di,
                                    hist, w.conv_w, w.conv_b, x->xs, w.x_w.h, w.x_w.l, x->dbc, R + 2 * NS, di, B,
                                    (int)(x->pos % 3)));
        else
            PROF(PC_CONV, flops, bytes,
                 hipLaunchKernelGGL((k_convx_step<2>), dim3((B + 15) / 16), dim3(256), lds, s, x->xz, (int64_t)2 * di,
                                    hist, w.conv_w, w.conv_b, x->xs, w.x_w.h, w.x_w.l, x->dbc, R + 2 * NS, di, B,
                                    (int)(x->pos % 3)));
    } else {
    // conv + SiLU -> xs
    PROF(PC_CONV, 8.0 * M * di, 4.0 * (2.0 * M * di + 6.0 * B * di),
         hipLaunchKernelGGL(k_conv_silu, dim3((di + 255) / 256, B), dim3(256), 0, s, x->xz, (int64_t)2 * di,
                            hist, w.conv_w, w.conv_b, x->xs, di, Tc, (int)(x->pos % 3)));
    // x_proj -> dbc [M][R+2NS]
    {
        PROF(PC_XPROJ, gemm_flops(M, R + 2 * NS, di), gemm_bytes(M, R + 2 * NS, di),
             rc = split ? launch_xproj(x->xs, M, di, w.x_w.h, w.x_w.l, x->dbc, R + 2 * NS, s)
                        : launch_xproj_f32(x->xs, M, di, w.x_w.f, x->dbc, R + 2 * NS, s));
        if (rc) return rc;
    }
    }
    }
    // dt_proj + softplus + scan + D + gate: y in place of xs (fp32) or split into ah/al
    if (part & 2) {
        float* ssm = x->ssm + ((int64_t)l * x->max_lanes + x->lane0) * di * NS;
        const double flops = (double)M * di * (2.0 * R + 6.0 * NS + 8.0);
        const double bytes = 4.0 * ((double)M * (3.0 * di + R + 2 * NS) + 2.0 * B * di * NS);
        if (R == 16) {
            if (split) PROF(PC_SCAN, flops, bytes, (launch_scan<16, 16, true>(x, w, ssm, B, Tc)));
            else PROF(PC_SCAN, flops, bytes, (launch_scan<16, 16, false>(x, w, ssm, B, Tc)));
        } else {
            if (split) PROF(PC_SCAN, flops, bytes, (launch_scan<16, 32, true>(x, w, ssm, B, Tc)));
            else PROF(PC_SCAN, flops, bytes, (launch_scan<16, 32, false>(x, w, ssm, B, Tc)));
        }
    }
    if (!(part & 4)) return BOA_OK;
    const bool ffn512 = split && d == ffn5::D && 4 * d == ffn5::DF && w.ff1_w.p && w.ff2_w.p;
    if (ffn512 && x->ffn_outp && w.out_w.p) {
        // out_proj + LN2 + FF1 + GELU + FF2 + residual in one kernel, d_model 512 (mm and the hidden layer kept
        // on chip)
        const double flops = gemm_flops(M, d, di) + gemm_flops(M, 4 * d, d) + gemm_flops(M, d, 4 * d);
        const double bytes = 4.0 * M * di + 4.0 * M * d * 2 + 2.0 * (w.ff1_w.l ? 2 : 1) * (2.0 * 4 * d * d + d * di);
        const unsigned grid = (unsigned)((M + ffn5::BM - 1) / ffn5::BM);
        if (w.ff1_w.l)
            PROF(PC_FFN, flops, bytes,
                 hipLaunchKernelGGL((k_ffn512<3, true>), dim3(grid), dim3(512), 0, s, nullptr, w.ln2_w, w.ln2_b,
                                    w.ff1_w.p, w.ff1_b, w.ff2_w.p, w.ff2_b, x->x, M, x->ah, x->al, w.out_w.p, w.out_b));
        else
            PROF(PC_FFN, flops, bytes,
                 hipLaunchKernelGGL((k_ffn512<2, true>), dim3(grid), dim3(512), 0, s, nullptr, w.ln2_w, w.ln2_b,
                                    w.ff1_w.p, w.ff1_b, w.ff2_w.p, w.ff2_b, x->x, M, x->ah, x->al, w.out_w.p, w.out_b));
        return BOA_OK;
    }
    // (fp32 mode included: its fragment-packed weights exist at d_model 256; its y is fp32 in place of xs)
    const bool ffn256 = d == ffn::D && 4 * d == ffn::DF && di == 2 * d && w.ff1_w.p && w.ff2_w.p;
    if (ffn256 && x->ffn_outp && w.out_w.p) {
        // out_proj + LN2 + FF1 + GELU + FF2 + residual in one kernel (mm and the hidden layer kept on chip)
        const double flops = gemm_flops(M, d, di) + gemm_flops(M, 4 * d, d) + gemm_flops(M, d, 4 * d);
        const double bytes = 4.0 * M * di + 4.0 * M * d * 2 + 2.0 * (w.ff1_w.l || !split ? 2 : 1) * (2.0 * 4 * d * d + d * di);
        const unsigned grid = (unsigned)((M + ffn::BM - 1) / ffn::BM);
        if (!split)
            PROF(PC_FFN, flops, bytes,
                 hipLaunchKernelGGL((k_ffn<1, true>), dim3(grid), dim3(512), 0, s, nullptr, w.ln2_w, w.ln2_b, w.ff1_w.p,
                                    w.ff1_b, w.ff2_w.p, w.ff2_b, x->x, M, reinterpret_cast<const uint16_t*>(x->xs),
                                    nullptr, w.out_w.p, w.out_b));
        else if (w.ff1_w.l)
            PROF(PC_FFN, flops, bytes,
                 hipLaunchKernelGGL((k_ffn<3, true>), dim3(grid), dim3(512), 0, s, nullptr, w.ln2_w, w.ln2_b, w.ff1_w.p,
                                    w.ff1_b, w.ff2_w.p, w.ff2_b, x->x, M, x->ah, x->al, w.out_w.p, w.out_b));
        else
            PROF(PC_FFN, flops, bytes,
                 hipLaunchKernelGGL((k_ffn<2, true>), dim3(grid), dim3(512), 0, s, nullptr, w.ln2_w, w.ln2_b, w.ff1_w.p,
                                    w.ff1_b, w.ff2_w.p, w.ff2_b, x->x, M, x->ah, x->al, w.out_w.p, w.out_b));
        return BOA_OK;
    }
    // out_proj -> mm [M][d]
    {
        GemmArgs g = gemm_args(x->xs, di, w.out_w, w.out_b, x->mm, d, M, d, di);
        if (split) {
            g.Ah = x->ah; g.Al = x->al;
            PROF(PC_OUT, gemm_flops(M, d, di), gemm_bytes(M, d, di), rc = (launch_gemm_bf<EPI_BIAS, true, false>(g, s)));
        } else {
            PROF(PC_OUT, gemm_flops(M, d, di), gemm_bytes(M, d, di), rc = (launch_gemm_f32<0, EPI_BIAS>(g, s)));
        }
        if (rc) return rc;
    }
    if (ffn512) {
        // LN2 + FF1 + GELU + FF2 + residual in one kernel, d_model 512 (hidden layer kept on chip)
        const double flops = gemm_flops(M, 4 * d, d) + gemm_flops(M, d, 4 * d);
        const double bytes = 4.0 * M * d * 3 + 2.0 * (w.ff1_w.l ? 2 : 1) * (2.0 * 4 * d * d);
        const unsigned grid = (unsigned)((M + ffn5::BM - 1) / ffn5::BM);
        if (w.ff1_w.l)
            PROF(PC_FFN, flops, bytes,
                 hipLaunchKernelGGL((k_ffn512<3, false>), dim3(grid), dim3(512), 0, s, x->mm, w.ln2_w, w.ln2_b,
                                    w.ff1_w.p, w.ff1_b, w.ff2_w.p, w.ff2_b, x->x, M, nullptr, nullptr, nullptr, nullptr));
        else
            PROF(PC_FFN, flops, bytes,
                 hipLaunchKernelGGL((k_ffn512<2, false>), dim3(grid), dim3(512), 0, s, x->mm, w.ln2_w, w.ln2_b,
                                    w.ff1_w.p, w.ff1_b, w.ff2_w.p, w.ff2_b, x->x, M, nullptr, nullptr, nullptr, nullptr));
        return BOA_OK;
    }
    if (ffn256) {
        // LN2 + FF1 + GELU + FF2 + residual in one kernel (hidden layer kept on chip)
        const double flops = gemm_flops(M, 4 * d, d) + gemm_flops(M, d, 4 * d);
        const double bytes = 4.0 * M * d * 3 + 2.0 * 2 * (2.0 * 4 * d * d);
        const unsigned grid = (unsigned)((M + ffn::BM - 1) / ffn::BM);
        if (!split)
            PROF(PC_FFN, flops, bytes,
                 hipLaunchKernelGGL((k_ffn<1, false>), dim3(grid), dim3(512), 0, s, x->mm, w.ln2_w, w.ln2_b, w.ff1_w.p,
                                    w.ff1_b, w.ff2_w.p, w.ff2_b, x->x, M, nullptr, nullptr, nullptr, nullptr));
        else if (w.ff1_w.l)
            PROF(PC_FFN, flops, bytes,
                 hipLaunchKernelGGL((k_ffn<3, false>), dim3(grid), dim3(512), 0, s, x->mm, w.ln2_w, w.ln2_b, w.ff1_w.p,
                                    w.ff1_b, w.ff2_w.p, w.ff2_b, x->x, M, nullptr, nullptr, nullptr, nullptr));
        else
            PROF(PC_FFN, flops, bytes,
                 hipLaunchKernelGGL((k_ffn<2, false>), dim3(grid), dim3(512), 0, s, x->mm, w.ln2_w, w.ln2_b, w.ff1_w.p,
                                    w.ff1_b, w.ff2_w.p, w.ff2_b, x->x, M, nullptr, nullptr, nullptr, nullptr));
        return BOA_OK;
    }
    // LN2 + FF1 + GELU -> g [M][4d]
    {
        GemmArgs g = gemm_args(x->mm, d, w.ff1_w, w.ff1_b, x->xz, 4 * d, M, 4 * d, d);
        if (split) {
            launch_ln_split(x, x->mm, M, w.ln2_w, w.ln2_b);
            g.Ah = x->ah; g.Al = x->al; g.Ch = gh; g.Cl = gl;
            PROF(PC_FF1, gemm_flops(M, 4 * d, d), gemm_bytes(M, 4 * d, d),
                 rc = (launch_gemm_bf<EPI_GELU, true, true>(g, s)));
        } else {
            launch_ln_stats(x, x->mm, d, M);
            g.ln_w = w.ln2_w; g.ln_b = w.ln2_b; g.ln_stats = x->stats;
            PROF(PC_FF1, gemm_flops(M, 4 * d, d), gemm_bytes(M, 4 * d, d),
                 rc = (d == 256) ? launch_gemm_f32<1, EPI_GELU>(g, s) : launch_gemm_f32<2, EPI_GELU>(g, s));
        }
        if (rc) return rc;
    }
    // FF2 + bias + block residual -> x
    {
        GemmArgs g = gemm_args(x->xz, 4 * d, w.ff2_w, w.ff2_b, x->x, d, M, d, 4 * d);
        g.R = x->x; g.ldr = d;
        if (split) {
            g.Ah = gh; g.Al = gl;
            PROF(PC_FF2, gemm_flops(M, d, 4 * d), gemm_bytes(M, d, 4 * d) + 4.0 * M * d,
                 rc = (launch_gemm_bf<EPI_RESID, true, false>(g, s)));
        } else {
            PROF(PC_FF2, gemm_flops(M, d, 4 * d), gemm_bytes(M, d, 4 * d) + 4.0 * M * d,
                 rc = (launch_gemm_f32<0, EPI_RESID>(g, s)));
        }
        if (rc) return rc;
    }
    return BOA_OK;
}

// Full model over B x Tc rows already embedded in ctx->x; logits to `out` (ld V).
// Head (Linear -> ReLU -> Linear) over B x Tc rows of ctx->x; logits to `out` (ld V).
static int run_head(boa_ctx* x, int B, int Tc, float* out) {
    const int d = x->d, V = x->V;
    const int64_t M = (int64_t)B * Tc;
    const bool split = x->prec != BOA_PREC_F32;
    int rc = 0;
    GemmArgs g1 = gemm_args(x->x, d, x->h1_w, x->h1_b, x->mm, d, M, d, d);
    GemmArgs g2 = gemm_args(x->mm, d, x->h2_w, x->h2_b, out, V, M, V, d);
    if (split) {
        g1.Ch = x->ah; g1.Cl = x->al;
        g2.Ah = x->ah; g2.Al = x->al;
        PROF(PC_HEAD1, gemm_flops(M, d, d), gemm_bytes(M, d, d),
             rc = (launch_gemm_bf<EPI_RELU, false, true>(g1, x->stream)));
        if (rc) return rc;
        PROF(PC_HEAD2, gemm_flops(M, V, d), gemm_bytes(M, V, d),
             rc = (launch_gemm_bf<EPI_BIAS, true, false>(g2, x->stream)));
    } else {
        PROF(PC_HEAD1, gemm_flops(M, d, d), gemm_bytes(M, d, d), rc = (launch_gemm_f32<0, EPI_RELU>(g1, x->stream)));
        if (rc) return rc;
        PROF(PC_HEAD2, gemm_flops(M, V, d), gemm_bytes(M, V, d), rc = (launch_gemm_f32<0, EPI_BIAS>(g2, x->stream)));
    }
    if (rc) return rc;
    BOA_HIP_TRY(hipGetLastError());
    return BOA_OK;
}

static int run_model(boa_ctx* x, int B, int Tc, float* out) {
    for (int l = 0; l < x->L; ++l) {
        const int rc = run_layer(x, l, B, Tc);
        if (rc) return rc;
    }
    return run_head(x, B, Tc, out);
}

// The context as seen by the launches of one group of the lanes on its own stream (the two-stream decode, the
// compress groups): the group's per-row activations start row_off rows into every workspace buffer (each holds
// max_rows rows at its widest row length, so any row length fits), its per-lane state starts at lane0, and it
// runs on stream s.  Restores the context on destruction.
struct LaneView {
    boa_ctx* x;
    float *px, *pxz, *pxs, *pdbc, *pmm, *plog;
    float2* pst;
    uint16_t *pah, *pal;
    int64_t pl0;
    hipStream_t ps;
    LaneView(boa_ctx* c, int64_t row_off, int64_t lane0, hipStream_t s)
        : x(c), px(c->x), pxz(c->xz), pxs(c->xs), pdbc(c->dbc), pmm(c->mm), plog(c->logits), pst(c->stats),
          pah(c->ah), pal(c->al), pl0(c->lane0), ps(c->stream) {
        if (row_off) {
            const int64_t hr = row_off;
            const int64_t d = x->d, di = x->di, V = x->V, W = x->R + 2 * x->NS;
            x->x += hr * d;
            x->xz += hr * std::max(2 * di, 4 * d);
            x->xs += hr * di;
            x->dbc += hr * W;
            x->mm += hr * d;
            x->logits += hr * V;
            x->stats += hr;
            if (x->ah) x->ah += hr * std::max(d, di);
            if (x->al) x->al += hr * std::max(d, di);
        }
        x->lane0 = lane0;
        x->stream = s;
    }
    ~LaneView() {
        x->x = px; x->xz = pxz; x->xs = pxs; x->dbc = pdbc; x->mm = pmm; x->logits = plog; x->stats = pst;
        x->ah = pah; x->al = pal; x->lane0 = pl0; x->stream = ps;
    }
};

static unsigned row_blocks(int64_t rows) { return (unsigned)((rows + 3) / 4); }  // 4 waves per 256-thread block

static void launch_embed_tokens(boa_ctx* x, const int32_t* tokens, int64_t tok_stride, int t0, int Tc, int64_t rows) {
    PROF(PC_EMBED, 0.0, 4.0 * rows * x->d,
         hipLaunchKernelGGL(k_embed_tokens, dim3(row_blocks(rows)), dim3(256), 0, x->stream, tokens, tok_stride, t0,
                            Tc, rows, x->emb, x->d, x->V, x->x));
}

// Arguments of one k_fused_step launch at the context's current position (logits and decode fields are
// filled in by the caller).
static FusedArgs fused_args(boa_ctx* x, int32_t lanes, const int32_t* tokens_in) {
    FusedArgs a;
    memset(&a, 0, sizeof(a));
    a.layers = x->d_layers; a.L = x->L; a.V = x->V; a.B = lanes; a.p0m3 = (int)(x->pos % 3);
    a.max_lanes = x->max_lanes;
    a.emb = x->emb; a.h1_b = x->h1_b; a.h2_b = x->h2_b; a.h1_p = x->h1_w.p; a.h2_p = x->h2_w.p;
    a.ssm = x->ssm; a.hist = x->conv_hist; a.tokens_in = tokens_in;
    a.scr = x->xz;  // per-lane scratch rows of the d_model 512 kernel (row = lane)
    a.nsteps = 1;
    return a;
}

static hipError_t launch_fused(const boa_ctx* x, const FusedArgs& a, hipStream_t s) {
    const int nt = x->prec == BOA_PREC_BF16X3 ? 3 : (x->prec == BOA_PREC_BF16W ? 2 : 1);
    return x->d == 512 ? launch_fused_step512(a, nt, s) : launch_fused_step(a, nt, s);
}

// Compulsory HBM bytes of one fused step: SSM state read + write, conv history (3 reads, 1 write), input
// embedding rows, per-lane coder state and bytes, plus the packed weights once (4 B per parameter as fp32
// or bf16 hi + lo, 2 B as bf16).
static double fused_bytes(const boa_ctx* x, int32_t lanes) {
    const double per_lane_layer = 2.0 * x->di * x->NS * 4 + 4.0 * x->di * 4;
    double wbytes = 0.0;
    for (const auto& w : x->layers)
        wbytes += 2.0 * (double)(w.in_w.n + w.x_w.n + w.out_w.n + w.ff1_w.n + w.ff2_w.n);
    wbytes += 2.0 * (double)(x->h1_w.n + x->h2_w.n);
    if (x->prec != BOA_PREC_BF16W) wbytes *= 2.0;
    return (double)lanes * (x->L * per_lane_layer + 4.0 * x->d + 64.0) + wbytes;
}

static double fused_flops(const boa_ctx* x, int32_t lanes) {
    double params = 0.0;
    for (const auto& w : x->layers)
        params += (double)(w.in_w.n + w.x_w.n + w.out_w.n + w.ff1_w.n + w.ff2_w.n);
    params += (double)(x->h1_w.n + x->h2_w.n);
    const double scan = (double)x->L * x->di * (2.0 * x->R + 6.0 * x->NS + 8.0);
    return (double)lanes * (2.0 * params + scan);
}

extern "C" int boa_model_step(boa_ctx* x, const int32_t* d_tokens, int32_t lanes, float* d_logits) {
    if (!x || !d_tokens || !d_logits || lanes < 1 || lanes > x->max_lanes)
        return boa_fail(BOA_ERR_ARG, "boa_model_step: bad arguments");
    if (x->fused) {
        FusedArgs a = fused_args(x, lanes, d_tokens);
        a.logits = d_logits;
        hipError_t e = hipSuccess;
        PROF(PC_FUSED, fused_flops(x, lanes), fused_bytes(x, lanes),
             e = launch_fused(x, a, x->stream));
        if (e != hipSuccess) return boa_fail_hip(e, "k_fused_step", __FILE__, __LINE__);
        x->pos += 1;
        return BOA_OK;
    }
    launch_embed_tokens(x, d_tokens, 1, 0, 1, lanes);
    const int rc = run_model(x, lanes, 1, d_logits);
    x->pos += 1;
    return rc;
}

extern "C" int boa_model_forward(boa_ctx* x, const int32_t* d_tokens, int64_t tok_stride, int32_t lanes, int32_t len,
                                 float* d_logits) {
    if (!x || !d_tokens || !d_logits || lanes < 1 || lanes > x->max_lanes || len < 0 || tok_stride < len)
        return boa_fail(BOA_ERR_ARG, "boa_model_forward: bad arguments");
    for (int t0 = 0; t0 < len; t0 += x->tile_len) {
        const int Tc = std::min(x->tile_len, len - t0);
        const int64_t rows = (int64_t)lanes * Tc;
        launch_embed_tokens(x, d_tokens, tok_stride, t0, Tc, rows);
        int rc = run_model(x, lanes, Tc, x->logits);
        x->pos += Tc;
        if (rc) return rc;
        hipLaunchKernelGGL(k_scatter_logits, dim3(row_blocks(rows)), dim3(256), 0, x->stream, x->logits, x->V, Tc, t0,
                           len, rows, d_logits);
    }
    BOA_HIP_TRY(hipGetLastError());
    return BOA_OK;
}

// The fused head + quantiser kernel covers full tiles of 64 positions, vocab 256, d_model 256 (every precision
// mode) or 512 (split modes), from fragment-packed head weights; other tiles take the head GEMMs and
// k_encode_tile (same values).
static bool head_xq_ok(const boa_ctx* x, int Tc) {
    return x->head_xq && Tc == headq::BM && x->V == headq::V && (x->d == 256 || (x->d == 512 && x->prec != BOA_PREC_F32)) &&
           x->h1_w.p && x->h2_w.p;
}

static int launch_head_xq(boa_ctx* x, int lanes, int t0, const uint8_t* bytes, int64_t stride, const int32_t* lens,
                          uint2* lf) {
    const int d = x->d, V = x->V;
    const int64_t M = (int64_t)lanes * headq::BM;
    const double flops = gemm_flops(M, d, d) + gemm_flops(M, V, d);
    const double bytes_ = 4.0 * M * d + 8.0 * M + (double)M + 2.0 * (x->prec == BOA_PREC_BF16W ? 1 : 2) * (double)(x->h1_w.n + x->h2_w.n);
    const bool three = x->prec == BOA_PREC_BF16X3;
    hipStream_t s = x->stream;
#define HXQ(NT, D)                                                                                                  \
    PROF(PC_HEADXQ, flops, bytes_,                                                                                  \
         hipLaunchKernelGGL((k_head_xq<NT, D>), dim3((unsigned)lanes), dim3(512), 0, s, x->x, x->h1_w.p, x->h1_b,    \
                            x->h2_w.p, x->h2_b, t0, bytes, stride, lens, lf))
    if (d == 256) {
        if (x->prec == BOA_PREC_F32) HXQ(1, 256); else if (three) HXQ(3, 256); else HXQ(2, 256);
    } else {
        if (three) HXQ(3, 512); else HXQ(2, 512);
    }
#undef HXQ
    BOA_HIP_TRY(hipGetLastError());
    return BOA_OK;
}

extern "C" int boa_compress(boa_ctx* x, const uint8_t* d_bytes, int64_t byte_stride, const int32_t* d_lens,
                            int32_t lanes, int32_t max_len, uint32_t* d_words, int64_t pitch_words, int32_t* d_nwords) {
    if (!x || !d_bytes || !d_lens || !d_words || !d_nwords || lanes < 1 || lanes > x->max_lanes || max_len < 1 ||
        byte_stride < max_len || pitch_words < 1)
        return boa_fail(BOA_ERR_ARG, "boa_compress: bad arguments");
    hipStream_t s = x->stream;
    int rc = boa_state_reset(x, lanes);
    if (rc) return rc;
    hipLaunchKernelGGL(k_enc_init, dim3((lanes + 255) / 256), dim3(256), 0, s, x->enc, lanes);
    BOA_HIP_TRY(hipMemsetAsync(x->flag, 0, sizeof(int32_t), s));
    const int positions = max_len - 1;  // model inputs 0..max_len-2 predict bytes 1..max_len-1
    // lane groups: group g holds lanes [lo[g], lo[g + 1]), its rows lo[g] * tile_len rows into the workspace
    const int G = x->stream3 ? 3 : 2;
    int lo[4];
    for (int g = 0; g <= G; ++g) lo[g] = (int)((int64_t)lanes * g / G);
    const bool halves = x->stream2 && x->compress_halves && lanes >= 256 * G;
    if (halves) {
        // Groups of the lanes on their own streams, each running its layers in order (per layer: the mixer input
        // kernel, the scan, the feed-forward kernel), so that the GPU interleaves the groups' kernels: a
        // VALU-bound scan of one beside the MFMA-bound kernels of another, or two of those.  Ordering the scans
        // to alternate between two halves (A's layer l after B's layer l - 1, B's after A's) measured 1.3% slower
        // than leaving the halves free.  Each group's arithmetic is unchanged.
        const int L = x->L;
        hipStream_t gs[3] = {s, x->stream2, x->stream3};
        hipEvent_t join[2] = {x->half_ev[2 * L], x->half_ev[2 * L + 1]};
        BOA_HIP_TRY(hipEventRecord(join[0], s));  // the other streams start after the coder initialisation
        for (int g = 1; g < G; ++g) BOA_HIP_TRY(hipStreamWaitEvent(gs[g], join[0], 0));
        for (int t0 = 0; t0 < positions; t0 += x->tile_len) {
            const int Tc = std::min(x->tile_len, positions - t0);
            const bool fuse_emb = embed_in_mixin(x, Tc);
            for (int g = 0; g < G && !fuse_emb; ++g) {
                LaneView v(x, (int64_t)lo[g] * x->tile_len, lo[g], gs[g]);
                const int64_t b0 = x->lane0, rows = (int64_t)(lo[g + 1] - lo[g]) * Tc;
                PROF(PC_EMBED, 0.0, 4.0 * rows * x->d,
                     hipLaunchKernelGGL(k_embed_bytes, dim3(row_blocks(rows)), dim3(256), 0, x->stream,
                                        d_bytes + b0 * byte_stride, byte_stride, d_lens + b0, t0, Tc, rows, x->emb,
                                        x->d, x->V, x->x));
            }
            for (int l = 0; l < L; ++l) {
                for (int g = 0; g < G; ++g) {
                    LaneView v(x, (int64_t)lo[g] * x->tile_len, lo[g], gs[g]);
                    const int64_t b0 = x->lane0;
                    EmbedFromBytes eb(x, fuse_emb && l == 0, d_bytes + b0 * byte_stride, byte_stride, d_lens + b0, t0);
                    rc = run_layer(x, l, lo[g + 1] - lo[g], Tc);
                    if (rc) return rc;
                }
            }
            for (int g = 0; g < G; ++g) {
                LaneView v(x, (int64_t)lo[g] * x->tile_len, lo[g], gs[g]);
                const int nl = lo[g + 1] - lo[g];
                const int64_t b0 = x->lane0, rows = (int64_t)nl * Tc;
                if (head_xq_ok(x, Tc)) {
                    uint2* lf = reinterpret_cast<uint2*>(x->logits);
                    rc = launch_head_xq(x, nl, t0, d_bytes + b0 * byte_stride, byte_stride, d_lens + b0, lf);
                    if (rc) return rc;
                    PROF(PC_ENCODE, 0.0, 8.0 * rows + 32.0 * nl,
                         hipLaunchKernelGGL(k_encode_lf, dim3((nl + 255) / 256), dim3(256), 0, x->stream, lf, Tc, nl,
                                            x->enc + b0, d_words + b0 * pitch_words, pitch_words));
                } else {
                    rc = run_head(x, nl, Tc, x->logits);
                    if (rc) return rc;
                    PROF(PC_ENCODE, 0.0, 4.0 * rows * x->V + (double)rows,
                         hipLaunchKernelGGL(k_encode_tile, dim3(nl), dim3(64), 0, x->stream, x->logits, x->V, Tc, t0,
                                            d_bytes + b0 * byte_stride, byte_stride, d_lens + b0, x->enc + b0,
                                            d_words + b0 * pitch_words, pitch_words));
                }
            }
            x->pos += Tc;
        }
        BOA_HIP_TRY(hipGetLastError());
        for (int g = 1; g < G; ++g) {  // the context's stream joins the others
            BOA_HIP_TRY(hipEventRecord(join[g - 1], gs[g]));
            BOA_HIP_TRY(hipStreamWaitEvent(s, join[g - 1], 0));
        }
    }
    for (int t0 = 0; !halves && t0 < positions; t0 += x->tile_len) {
        const int Tc = std::min(x->tile_len, positions - t0);
        const int64_t rows = (int64_t)lanes * Tc;
        const bool fuse_emb = embed_in_mixin(x, Tc);
        if (!fuse_emb)
            PROF(PC_EMBED, 0.0, 4.0 * rows * x->d,
                 hipLaunchKernelGGL(k_embed_bytes, dim3(row_blocks(rows)), dim3(256), 0, s, d_bytes, byte_stride, d_lens,
                                    t0, Tc, rows, x->emb, x->d, x->V, x->x));
        if (head_xq_ok(x, Tc)) {
            // layers, then head + quantiser in one kernel (logits on chip) and the sequential coder
            for (int l = 0; l < x->L && !rc; ++l) {
                EmbedFromBytes eb(x, fuse_emb && l == 0, d_bytes, byte_stride, d_lens, t0);
                rc = run_layer(x, l, lanes, Tc);
            }
            x->pos += Tc;
            if (rc) return rc;
            uint2* lf = reinterpret_cast<uint2*>(x->logits);  // (lo, width) per position: 8 of the row's V * 4 bytes
            rc = launch_head_xq(x, lanes, t0, d_bytes, byte_stride, d_lens, lf);
            if (rc) return rc;
            PROF(PC_ENCODE, 0.0, 8.0 * rows + 32.0 * lanes,
                 hipLaunchKernelGGL(k_encode_lf, dim3((lanes + 255) / 256), dim3(256), 0, s, lf, Tc, lanes, x->enc,
                                    d_words, pitch_words));
            continue;
        }
        {
            EmbedFromBytes eb(x, fuse_emb, d_bytes, byte_stride, d_lens, t0);  // used by layer 0 only
            rc = run_model(x, lanes, Tc, x->logits);
        }
        x->pos += Tc;
        if (rc) return rc;
        PROF(PC_ENCODE, 0.0, 4.0 * rows * x->V + (double)rows,
             hipLaunchKernelGGL(k_encode_tile, dim3(lanes), dim3(64), 0, s, x->logits, x->V, Tc, t0, d_bytes,
                                byte_stride, d_lens, x->enc, d_words, pitch_words));
    }
    hipLaunchKernelGGL(k_enc_finish, dim3((lanes + 255) / 256), dim3(256), 0, s, x->enc, d_words, pitch_words, d_nwords,
                       x->flag, lanes);
    BOA_HIP_TRY(hipGetLastError());
    int32_t flag = 0;
    BOA_HIP_TRY(hipMemcpyAsync(&flag, x->flag, sizeof(int32_t), hipMemcpyDeviceToHost, s));
    BOA_HIP_TRY(hipStreamSynchronize(s));
    if (flag) return boa_fail(BOA_ERR_OVERFLOW, "boa_compress: a stream exceeded pitch_words=%lld", (long long)pitch_words);
    return BOA_OK;
}

extern "C" int boa_decompress(boa_ctx* x, const uint32_t* d_payload, int64_t payload_words, const int64_t* d_word_off,
                              const int32_t* d_nwords, const uint8_t* d_first, const int32_t* d_lens, int32_t lanes,
                              int32_t max_len, uint8_t* d_out, int64_t out_stride) {
    if (!x || !d_payload || payload_words < 0 || !d_word_off || !d_nwords || !d_first || !d_lens || !d_out ||
        lanes < 1 || lanes > x->max_lanes || max_len < 1 || out_stride < max_len)
        return boa_fail(BOA_ERR_ARG, "boa_decompress: bad arguments");
    hipStream_t s = x->stream;
    int rc = boa_state_reset(x, lanes);
    if (rc) return rc;
    hipLaunchKernelGGL(k_dec_init, dim3((lanes + 255) / 256), dim3(256), 0, s, x->dec, d_payload, payload_words,
                       d_word_off, d_nwords, d_first, d_lens, x->tokens, d_out, out_stride, lanes);
    if (x->fused) {
        // the fused kernel runs fused_steps positions per launch, feeding each decoded byte back itself
        for (int t = 1; t < max_len; t += x->fused_steps) {
            FusedArgs a = fused_args(x, lanes, x->tokens);
            a.decode = 1; a.t = t; a.nsteps = std::min(x->fused_steps, max_len - t); a.stagger_us = x->stagger_us;
            a.stagger_classes = x->stagger_classes;
            a.lens = d_lens; a.dec = x->dec; a.payload = d_payload; a.payload_words = payload_words;
            a.off = d_word_off; a.nwords = d_nwords; a.tokens_out = x->tokens; a.out = d_out; a.out_stride = out_stride;
            hipError_t e = hipSuccess;
            PROF(PC_FUSED, a.nsteps * fused_flops(x, lanes), a.nsteps * fused_bytes(x, lanes),
                 e = launch_fused(x, a, s));
            if (e != hipSuccess) return boa_fail_hip(e, "k_fused_step", __FILE__, __LINE__);
            x->pos += a.nsteps;
        }
        BOA_HIP_TRY(hipStreamSynchronize(s));
        return BOA_OK;
    }
    if (x->stream2 && lanes >= 512) {
        // Two halves of the lanes on two streams.  Per layer and half: LN1 + in_proj, then conv + scan (the
        // state traffic), then out_proj + feed-forward.  The state groups alternate between the halves (A's
        // layer l after B's layer l - 1, B's layer l after A's layer l), so one half's HBM-bound scan runs
        // beside the other half's GEMMs.  Each half's arithmetic is unchanged.  (configs[4], 16384 lanes:
        // 12.96 ms per step on one stream, 12.14 alternating, 12.34 with the halves left to run freely.)
        const int L = x->L, la = lanes / 2, lb = lanes - la;
        hipEvent_t* evA = x->half_ev.data();
        hipEvent_t* evB = evA + L;
        hipEvent_t join = evA[2 * L];
        BOA_HIP_TRY(hipEventRecord(join, s));  // the second stream starts after the decoder initialisation
        BOA_HIP_TRY(hipStreamWaitEvent(x->stream2, join, 0));
        for (int t = 1; t < max_len; ++t) {
            for (int h = 0; h < 2; ++h) {
                LaneView v(x, h ? x->max_rows / 2 : 0, h ? la : 0, h ? x->stream2 : s);
                launch_embed_tokens(x, x->tokens + x->lane0, 1, 0, 1, h ? lb : la);
            }
            for (int l = 0; l < L; ++l) {
                for (int h = 0; h < 2; ++h) {
                    LaneView v(x, h ? x->max_rows / 2 : 0, h ? la : 0, h ? x->stream2 : s);
                    const int nl = h ? lb : la;
                    rc = run_layer(x, l, nl, 1, 1);
                    if (rc) return rc;
                    hipEvent_t prev = h ? evA[l] : (l > 0 ? evB[l - 1] : (t > 1 ? evB[L - 1] : nullptr));
                    if (prev) BOA_HIP_TRY(hipStreamWaitEvent(x->stream, prev, 0));
                    rc = run_layer(x, l, nl, 1, 2);
                    if (rc) return rc;
                    BOA_HIP_TRY(hipEventRecord(h ? evB[l] : evA[l], x->stream));
                    rc = run_layer(x, l, nl, 1, 4);
                    if (rc) return rc;
                }
            }
            for (int h = 0; h < 2; ++h) {
                LaneView v(x, h ? x->max_rows / 2 : 0, h ? la : 0, h ? x->stream2 : s);
                const int nl = h ? lb : la;
                const int64_t b0 = x->lane0;
                rc = run_head(x, nl, 1, x->logits);
                if (rc) return rc;
                PROF(PC_DECODE, 0.0, 4.0 * nl * x->V + (double)nl,
                     hipLaunchKernelGGL(k_decode_step, dim3(nl), dim3(64), 0, x->stream, x->logits, x->V, t,
                                        d_lens + b0, x->dec + b0, d_payload, payload_words, d_word_off + b0,
                                        d_nwords + b0, x->tokens + b0, d_out + b0 * out_stride, out_stride));
            }
            x->pos += 1;
        }
        BOA_HIP_TRY(hipGetLastError());
        BOA_HIP_TRY(hipEventRecord(join, x->stream2));  // the context's stream joins the second
        BOA_HIP_TRY(hipStreamWaitEvent(s, join, 0));
        BOA_HIP_TRY(hipStreamSynchronize(s));
        return BOA_OK;
    }
    for (int t = 1; t < max_len; ++t) {
        launch_embed_tokens(x, x->tokens, 1, 0, 1, lanes);
        rc = run_model(x, lanes, 1, x->logits);
        x->pos += 1;
        if (rc) return rc;
        PROF(PC_DECODE, 0.0, 4.0 * lanes * x->V + (double)lanes,
             hipLaunchKernelGGL(k_decode_step, dim3(lanes), dim3(64), 0, s, x->logits, x->V, t, d_lens, x->dec,
                                d_payload, payload_words, d_word_off, d_nwords, x->tokens, d_out, out_stride));
    }
    BOA_HIP_TRY(hipGetLastError());
    BOA_HIP_TRY(hipStreamSynchronize(s));
    return BOA_OK;
}
