// Fused decompress steps for d_model 512 (configs[4]'s shape: d_inner 1024, d_state 16, dt_rank 32, x_proj width
// 64, vocab 256): the whole model for 32 chunk lanes per workgroup, many positions per launch, each decoded byte
// fed back as the next position's input without leaving the workgroup.
//
// Reference: the per-step loop of codec.py:211-323 (decompress_GPU: model.step on the batch of streams, softmax,
// table, coder.decode_step) and of portability_solved_cpp/boa.cpp:556-569 (step_batch +
// gpu_rc_decode_fused_step_batch), for the d_model 512 configuration.
//
// Design (gfx950).  At d_model 512 the activations of 16 lanes alone exceed the LDS (in_proj output 128 KB, FF
// hidden 128 KB), so everything wide is processed in 128-column chunks:
//   - 512 threads (8 waves) own 32 lanes: two M fragments per fragment-packed weight block, so the weights are
//     streamed from L2 once per 32 lanes;
//   - LDS: an operand buffer [32][512] bf16 hi/lo (64 KB; LN outputs, then dbc, staged y, mm and logits in fp32),
//     a chunk buffer [32][128] hi/lo (16 KB) and the residual stream [32][512] fp32 (66 KB with its row padding);
//   - per-lane scratch in device memory (the context's workspace rows, row = lane): z and the conv output xs (then
//     y in its place) between passes.  (The residual stream moved from these rows into LDS: 10.6 -> 10.3 ms per
//     step at 16384 lanes, 1.6 GB less scratch traffic per step.)
// Per layer: LN1 -> in_proj in 16 chunks (z chunks to scratch; x chunks: conv + SiLU with the history ring, xs to
// scratch, x_proj partials of the chunk's two 64-channel K blocks folded into dbc in registers) -> dbc to LDS ->
// scan pass (dt_proj + softplus + selective scan + D + gate; the state of 8 rows in flight per thread) -> out_proj
// over y staged in two K halves -> mm -> LN2 -> feed-forward in 16 hidden chunks (FF1 + GELU into the chunk
// buffer, FF2 accumulated) -> residual.  Head (two chunked GEMMs) -> quantiser + range decoder.
// Every output accumulates its K steps in ascending order with the same split-product sequence as the tiled and
// compress-tile kernels, x_proj is the same left fold of 64-channel K-block partials, and every elementwise step
// calls the same device function (model_dev.h), so the logits equal those of the compress path bit for bit.
#include "model_dev.h"
#include "model_internal.h"

namespace boa {

namespace {

constexpr int D = 512;              // d_model
constexpr int DI = 1024;            // d_inner
constexpr int NS = 16;              // d_state
constexpr int R = 32;               // dt_rank
constexpr int FW = R + 2 * NS;      // x_proj width (dt | B | C) = 64
constexpr int VV = 256;             // vocab
constexpr int ROWS = 32;            // lanes per workgroup
constexpr int MF = ROWS / 16;       // M fragments per weight block
constexpr int NTHR = 512;           // 8 waves
constexpr int NWAVE = NTHR / 64;
constexpr int CH = 128;             // chunk width (channels, hidden units)
constexpr int NFC = 8 / NWAVE;      // fragments per wave of a 128-column chunk GEMM (in_proj, FF1, head1)
constexpr int NFO = 32 / NWAVE;     // fragments per wave of a 512-output GEMM (out_proj, FF2)
constexpr int NFH = 16 / NWAVE;     // fragments per wave of head2 (256 outputs)
constexpr int KSD = D / 32;         // K steps over d_model
constexpr int RPW = ROWS / NWAVE;   // rows per wave (embedding, LN, decode)
constexpr int RPT = ROWS * CH / NTHR;  // rows per thread in the scan pass
constexpr int LLOG = VV + 4;        // logits row stride (fp32)
constexpr int SZ_A = 2 * ROWS * D * 2;    // operand [2][ROWS][D] bf16 (64 KB); fp32 views: dbc, y, mm, logits
constexpr int SZ_C = 2 * ROWS * CH * 2;   // chunk operand [2][ROWS][CH] bf16 (16 KB)
constexpr int LRS = D + 4;                // residual rows (fp32): 4 mod 64 words, so the column-wise residual
                                          // update (16 lanes of 4 rows) touches distinct banks
constexpr int SZ_R = ROWS * LRS * 4;      // residual stream [ROWS][LRS] fp32 (66 KB)
static_assert(SZ_A + SZ_C + SZ_R <= 160 * 1024, "LDS budget");
static_assert(ROWS * LLOG * 4 <= SZ_A && ROWS * D * 4 <= SZ_A && ROWS * FW * 4 <= SZ_A, "fp32 views fit");
static_assert(NFC >= 1 && NFO * NWAVE == 32 && NFH * NWAVE == 16 && 4 * MF == NWAVE, "wave mapping");

// 16-byte chunks of a row XOR-swizzled by the row's low 4 bits: 16-row fragment reads spread over the banks
__device__ __forceinline__ int a_off(int r, int k) { return r * D + (((k >> 3) ^ (r & 15)) << 3) + (k & 7); }
__device__ __forceinline__ int c_off(int r, int k) { return r * CH + (((k >> 3) ^ (r & 15)) << 3) + (k & 7); }

// Per-lane scratch rows (z, xs, y): 16-byte stores, 4- and 16-byte loads with the default cache policy.  Each
// value is read back a phase later by this workgroup; with the non-temporal policy (streamed past L2) the decode
// step measured 7% slower (11.06 against 10.32 ms at 16384 lanes), so the rows stay cacheable.
__device__ __forceinline__ void scr_st16(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(bufv4, v), r, off, 0, 0);
}
__device__ __forceinline__ void scr_st1(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off, 0, 0);
}
__device__ __forceinline__ float scr_ld1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ u32x4 scr_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

template <int NT>
__device__ __forceinline__ u32x4 wblk_lo(gptr<uint16_t> q, u32x4 hi) {
    if constexpr (NT == 3) return ldg16(q + 512);
    return hi;
}

typedef __attribute__((address_space(4))) const FusedArgs KArgs;

// Lane-derived indices from an opaque copy of the lane index, declared at the top of each phase or chunk: derived
// LDS and memory offsets are then formed where they are used instead of being hoisted out of the layer and step
// loops, where dozens of them would stay live (and spill) across every phase.
#define LANE_VARS                                   \
    int lq_ = lane;                                 \
    __asm__ volatile("" : "+v"(lq_));               \
    const int ar = lq_ & 15, kq = 8 * (lq_ >> 4);   \
    const int m_of = 4 * (lq_ >> 4), l4 = 4 * lq_;  \
    (void)ar; (void)kq; (void)m_of; (void)l4;
// The layer's parameter table entry and the scratch descriptors, re-formed per phase from opaque copies (uniform
// values held across all phases would exhaust the scalar registers).
#define LAYER_VARS                            \
    const FusedLayer* wl_ = a.layers + l;     \
    __asm__ volatile("" : "+s"(wl_));         \
    const FusedLayer& w = *wl_;
#define SCR_VARS                                                                                   \
    int64_t b0_ = b0;                                                                              \
    __asm__ volatile("" : "+s"(b0_));                                                              \
    const __amdgpu_buffer_rsrc_t rscr = buf_rsrc(a.scr + b0_ * 2 * DI, (uint32_t)nb * 2 * DI * 4); \
    (void)rscr;

// acc[n][m] += A[16 m + .., K step s] x W^T for this wave's NFC fragments of a chunk GEMM, the weight block as the
// MFMA A operand (lane l holds row 16 m + l % 16, columns 16 f + 4 (l / 16) .. + 3)
template <int NT>
__device__ __forceinline__ void chunk_kstep(floatx4 (&acc)[NFC][MF], const uint16_t* sAh, const uint16_t* sAl, int s,
                                            int arq, int kqq, const u32x4 (&bh)[NFC], const u32x4 (&bl)[NFC]) {
    bf16x8 ah[MF], al[MF];
#pragma unroll
    for (int m = 0; m < MF; ++m) {
        const int o = a_off(16 * m + arq, 32 * s + kqq);
        ah[m] = *reinterpret_cast<const bf16x8*>(sAh + o);
        al[m] = *reinterpret_cast<const bf16x8*>(sAl + o);
    }
#pragma unroll
    for (int n = 0; n < NFC; ++n)
#pragma unroll
        for (int m = 0; m < MF; ++m)
            acc[n][m] = mfma_split_step_t<NT>(acc[n][m], ah[m], al[m], __builtin_bit_cast(bf16x8, bh[n]),
                                              __builtin_bit_cast(bf16x8, bl[n]));
}

template <int NT>
__global__ void __launch_bounds__(NTHR, 1) k_fused_step512(FusedArgs a0) {
    constexpr int BLK = (NT == 3) ? 1024 : 512;  // uint16 elements per packed block (hi [+ lo])
    constexpr int DK = 4;                         // K steps in flight (in_proj, FF1)
    constexpr int DB = NFO;                       // blocks in flight (out_proj, FF2): one K step
    constexpr int PF = 8;                         // rows of recurrent state in flight per thread (scan)
    __shared__ __attribute__((aligned(16))) unsigned char lds[SZ_A + SZ_C + SZ_R];
    uint16_t* sAh = reinterpret_cast<uint16_t*>(lds);
    uint16_t* sAl = sAh + ROWS * D;
    uint16_t* sCh = reinterpret_cast<uint16_t*>(lds + SZ_A);
    uint16_t* sCl = sCh + ROWS * CH;
    float* sF = reinterpret_cast<float*>(lds);  // fp32 view of the operand buffer
    float* sRes = reinterpret_cast<float*>(lds + SZ_A + SZ_C);  // residual stream [ROWS][LRS]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t b0 = (int64_t)blockIdx.x * ROWS;
    const int nb = (int)((a0.B - b0) < ROWS ? (a0.B - b0) : ROWS);  // valid lanes of this workgroup
    // tokens of this wave's rows RPW wave + q (embedding and decode rows): lane q holds row q's token
    int tokv = (lane < RPW && RPW * wave + lane < nb) ? a0.tokens_in[b0 + RPW * wave + lane] : 0;
    int maxlen = 0;
    if (a0.decode)
        for (int r = 0; r < nb; ++r) maxlen = a0.lens[b0 + r] > maxlen ? a0.lens[b0 + r] : maxlen;
    int p0m3 = a0.p0m3;

#pragma unroll 1
    for (int step = 0; step < a0.nsteps; ++step) {
    // kernel arguments through an opaque pointer (kept out of SGPRs across the step loop)
    auto kp = (__attribute__((address_space(4))) const char*)__builtin_amdgcn_kernarg_segment_ptr();
    __asm__ volatile("" : "+s"(kp));
    KArgs& a = *reinterpret_cast<KArgs*>(kp);
    const int t = a.t + step;
    if (a.decode && t >= maxlen) break;  // every lane of this workgroup is complete (uniform)
    const int s1 = p0m3 == 2 ? 0 : p0m3 + 1, s2 = p0m3 == 0 ? 2 : p0m3 - 1;

    // ---- embedding (model.py:97): residual rows of this wave (LN1 reads only its own wave's rows: no barrier)
    {
        LANE_VARS
#pragma unroll
        for (int q = 0; q < RPW; ++q) {
            const int r = RPW * wave + q;
            int tk = __builtin_amdgcn_readlane(tokv, q);
            tk = tk < 0 ? 0 : (tk >= a.V ? a.V - 1 : tk);
            const gptr<float> e = G(a.emb) + (int64_t)tk * D;
            *reinterpret_cast<float4*>(sRes + r * LRS + l4) = ldg_f4(e + l4);
            *reinterpret_cast<float4*>(sRes + r * LRS + 256 + l4) = ldg_f4(e + 256 + l4);
        }
    }

#pragma unroll 1
    for (int l = 0; l < a.L; ++l) {
        // ---- LN1 of this wave's rows (ln_stats_row<2> layout: lane j holds 4j.. and 256 + 4j..) -> operand
        {
            LANE_VARS
            LAYER_VARS
            u32x4 ru[RPW][2];
#pragma unroll
            for (int q = 0; q < RPW; ++q) {
                ru[q][0] = *reinterpret_cast<const u32x4*>(sRes + (RPW * wave + q) * LRS + l4);
                ru[q][1] = *reinterpret_cast<const u32x4*>(sRes + (RPW * wave + q) * LRS + 256 + l4);
            }
            const float4 w0 = ldg_f4(G(w.ln1_w) + l4), w1 = ldg_f4(G(w.ln1_w) + 256 + l4);
            const float4 c0 = ldg_f4(G(w.ln1_b) + l4), c1 = ldg_f4(G(w.ln1_b) + 256 + l4);
            const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
            const float bv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
            for (int q = 0; q < RPW; ++q) {
                const int r = RPW * wave + q;
                const u32x4 u0 = ru[q][0], u1 = ru[q][1];
                const float v[8] = {__uint_as_float(u0.x), __uint_as_float(u0.y), __uint_as_float(u0.z),
                                    __uint_as_float(u0.w), __uint_as_float(u1.x), __uint_as_float(u1.y),
                                    __uint_as_float(u1.z), __uint_as_float(u1.w)};
                float mu, rs;
                ln_stats_row<2>(v, mu, rs);
                float y[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) y[i] = ln_apply(v[i], mu, rs, wv[i], bv[i]);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    uint2 hp, lp;
                    split4(y[4 * h], y[4 * h + 1], y[4 * h + 2], y[4 * h + 3], hp, lp);
                    const int o = a_off(r, 256 * h + l4);
                    *reinterpret_cast<uint2*>(sAh + o) = hp;
                    *reinterpret_cast<uint2*>(sAl + o) = lp;
                }
            }
        }
        __syncthreads();

        // ---- in_proj in 16 chunks of 128 columns: z chunks (8..15) first, then x chunks (0..7).  Wave w computes
        //      fragments 8 k + NFC w + n of chunk k for both M fragments; the blocks stream through a ring of DK K
        //      steps that runs on into the next chunk.  x_proj: wave w owns output fragment w % 4 of rows
        //      16 (w / 4) .. + 15, the left fold of the 64-channel K-block partials in a register.
        floatx4 dbc = floatx4{0.f, 0.f, 0.f, 0.f};
        {
            LAYER_VARS
            const gptr<uint16_t> wip = G(w.in_p);
            auto chunk_of = [](int i) { return i < 8 ? 8 + i : i - 8; };
            u32x4 rh[DK][NFC], rl[DK][NFC];
            auto issue = [&](int k, int s) {
#pragma unroll
                for (int n = 0; n < NFC; ++n) {
                    const gptr<uint16_t> q = wip + ((int64_t)(8 * k + NFC * wave + n) * KSD + s) * BLK + lane * 8;
                    rh[s % DK][n] = ldg16(q);
                    rl[s % DK][n] = wblk_lo<NT>(q, rh[s % DK][n]);
                }
            };
#pragma unroll
            for (int s = 0; s < DK; ++s) issue(chunk_of(0), s);
#pragma unroll 1
            for (int ci = 0; ci < 16; ++ci) {
                LANE_VARS
                SCR_VARS
                const int k = chunk_of(ci), kn = chunk_of(ci + 1 < 16 ? ci + 1 : ci);
                float4 bias[NFC];
#pragma unroll
                for (int n = 0; n < NFC; ++n) bias[n] = ldg_f4(G(w.in_b) + 16 * (8 * k + NFC * wave + n) + m_of);
                floatx4 acc[NFC][MF];
#pragma unroll
                for (int n = 0; n < NFC; ++n)
#pragma unroll
                    for (int m = 0; m < MF; ++m) acc[n][m] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < KSD; ++s) {
                    chunk_kstep<NT>(acc, sAh, sAl, s, ar, kq, rh[s % DK], rl[s % DK]);
                    if (s + DK < KSD) issue(k, s + DK);
                    else issue(kn, s + DK - KSD);  // (the last chunk reloads its own blocks, unused)
                    pin_loads();
                }
                float v[NFC][MF][4];
#pragma unroll
                for (int n = 0; n < NFC; ++n) {
                    const float bb[4] = {bias[n].x, bias[n].y, bias[n].z, bias[n].w};
#pragma unroll
                    for (int m = 0; m < MF; ++m)
#pragma unroll
                        for (int i = 0; i < 4; ++i) v[n][m][i] = epi_value<EPI_BIAS>(acc[n][m][i], bb[i]);
                }
                if (k >= 8) {
                    // z chunk: to scratch columns 0 .. 1023
#pragma unroll
                    for (int n = 0; n < NFC; ++n)
#pragma unroll
                        for (int m = 0; m < MF; ++m)
                            scr_st16(rscr, (uint32_t)((16 * m + ar) * 2 * DI + 16 * (8 * (k - 8) + NFC * wave + n) + m_of) * 4,
                                     f32x4{v[n][m][0], v[n][m][1], v[n][m][2], v[n][m][3]});
                    continue;
                }
                // x chunk k: causal conv + SiLU of channels 128 k + 16 (NFC w + n) + m_of .. + 3 of rows 16 m + ar
                {
                    const __amdgpu_buffer_rsrc_t hr =
                        buf_rsrc(a.hist + ((int64_t)l * a.max_lanes + b0) * 3 * DI, (uint32_t)nb * 3 * DI * 4);
#pragma unroll
                    for (int n = 0; n < NFC; ++n) {
                        const int cl = 16 * (NFC * wave + n) + m_of;  // first channel within the chunk
                        const int c = CH * k + cl;
                        f32x4 hh[MF][3];
#pragma unroll
                        for (int m = 0; m < MF; ++m) {
                            const uint32_t o = (uint32_t)((16 * m + ar) * 3 * DI + c) * 4;
                            hh[m][0] = buf_ld4(hr, o + p0m3 * DI * 4);
                            hh[m][1] = buf_ld4(hr, o + s1 * DI * 4);
                            hh[m][2] = buf_ld4(hr, o + s2 * DI * 4);
                        }
                        float4 cw[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i) cw[i] = ldg_f4(G(w.conv_w) + 4 * (c + i));
                        const float4 cb = ldg_f4(G(w.conv_b) + c);
                        const float cbv[4] = {cb.x, cb.y, cb.z, cb.w};
#pragma unroll
                        for (int m = 0; m < MF; ++m) {
                            const int r = 16 * m + ar;
                            const uint32_t o = (uint32_t)(r * 3 * DI + c) * 4;
                            float y[4];
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                y[i] = conv_point(cw[i], cbv[i], hh[m][0][i], hh[m][1][i], hh[m][2][i], v[n][m][i]);
                            buf_st4(hr, o + p0m3 * DI * 4, f32x4{v[n][m][0], v[n][m][1], v[n][m][2], v[n][m][3]});
                            scr_st16(rscr, (uint32_t)(r * 2 * DI + DI + c) * 4, f32x4{y[0], y[1], y[2], y[3]});
                            uint2 hp, lp;
                            split4(y[0], y[1], y[2], y[3], hp, lp);
                            const int oc = c_off(r, cl);
                            *reinterpret_cast<uint2*>(sCh + oc) = hp;
                            *reinterpret_cast<uint2*>(sCl + oc) = lp;
                        }
                    }
                }
                __syncthreads();
                // x_proj partials of K blocks 2 k and 2 k + 1 (64 channels each, two K steps from zero), output
                // fragment w % 4 of M fragment w / 4, folded in order into dbc
                {
                    const gptr<uint16_t> wxp = G(w.x_p);
                    const int xf = wave & 3, xm = wave >> 2;
                    u32x4 xb[4][2];
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        const gptr<uint16_t> q = wxp + ((int64_t)xf * (DI / 32) + 4 * k + s) * BLK + lane * 8;
                        xb[s][0] = ldg16(q);
                        xb[s][1] = wblk_lo<NT>(q, xb[s][0]);
                    }
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb) {
                        floatx4 part = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int s = 0; s < 2; ++s) {
                            const int o = c_off(16 * xm + ar, 64 * kb + 32 * s + kq);
                            const bf16x8 ah = *reinterpret_cast<const bf16x8*>(sCh + o);
                            const bf16x8 al = *reinterpret_cast<const bf16x8*>(sCl + o);
                            part = mfma_split_step<NT>(part, ah, al, __builtin_bit_cast(bf16x8, xb[2 * kb + s][0]),
                                                       __builtin_bit_cast(bf16x8, xb[2 * kb + s][1]));
                        }
                        dbc = (k == 0 && kb == 0) ? part : dbc + part;
                    }
                }
                __syncthreads();  // the next x chunk rewrites the chunk buffer
            }
        }
        // ---- dbc [ROWS][FW] fp32 into the operand buffer (its LN1 operand is dead)
        {
            LANE_VARS
#pragma unroll
            for (int i = 0; i < 4; ++i) sF[(16 * (wave >> 2) + m_of + i) * FW + 16 * (wave & 3) + ar] = dbc[i];
        }
        __syncthreads();

        // ---- scan pass in 8 chunks of 128 channels: thread = (channel c_in, rows RPT rh .. RPT rh + RPT - 1).  The
        //      state of PF rows is in flight at once (a register ring: the rows are independent).  y (fp32) replaces
        //      xs in the scratch row.
        {
            LAYER_VARS
            SCR_VARS
            const int c_in = tid & (CH - 1), rh = tid >> 7;
            const __amdgpu_buffer_rsrc_t sr =
                buf_rsrc(a.ssm + ((int64_t)l * a.max_lanes + b0) * DI * NS, (uint32_t)nb * DI * NS * 4);
#pragma unroll 1
            for (int q = 0; q < DI / CH; ++q) {
                int cq = CH * q + c_in;  // channel; opaque so per-row offsets are formed in each iteration
                __asm__ volatile("" : "+v"(cq));
                auto h_off = [&](int row, int n) { return (uint32_t)((row * NS / 4 + n / 4) * DI + cq) * 16; };
                f32x4 hs[PF][NS / 4];
                float zs[PF], xv[PF];
                auto load_row = [&](int r, int slot) {
                    const int row = RPT * rh + r;
#pragma unroll
                    for (int n = 0; n < NS; n += 4) hs[slot][n / 4] = buf_ld4(sr, h_off(row, n));
                    zs[slot] = scr_ld1(rscr, (uint32_t)(row * 2 * DI + cq) * 4);
                    xv[slot] = scr_ld1(rscr, (uint32_t)(row * 2 * DI + DI + cq) * 4);
                };
                // per-channel parameters, then the first rows' state (all independent loads)
                float av[NS];
#pragma unroll
                for (int n = 0; n < NS; n += 4) {
                    const float4 p = ldg_f4(G(w.Aneg) + ((int64_t)(n / 4) * DI + cq) * 4);
                    av[n] = p.x; av[n + 1] = p.y; av[n + 2] = p.z; av[n + 3] = p.w;
                }
                u32x4 wq[R / 4];
#pragma unroll
                for (int r = 0; r < R; r += 4) wq[r / 4] = ldg16(G(w.dt_w) + (int64_t)cq * R + r);
                const float bdt = G(w.dt_b)[cq], Dc = G(w.D)[cq];
#pragma unroll
                for (int r = 0; r < PF - 1 && r < RPT; ++r) load_row(r, r);
                pin_loads();
                float dtv[RPT];
                {
                    float wr[R];
#pragma unroll
                    for (int r = 0; r < R; r += 4) {
                        wr[r] = __uint_as_float(wq[r / 4].x); wr[r + 1] = __uint_as_float(wq[r / 4].y);
                        wr[r + 2] = __uint_as_float(wq[r / 4].z); wr[r + 3] = __uint_as_float(wq[r / 4].w);
                    }
#pragma unroll
                    for (int r = 0; r < RPT; ++r) dtv[r] = scan_dt<R>(sF + (RPT * rh + r) * FW, wr, bdt);
                }
#pragma unroll
                for (int r = 0; r < RPT; ++r) {
                    if (r + PF - 1 < RPT) load_row(r + PF - 1, (r + PF - 1) % PF);
                    pin_loads();
                    const int row = RPT * rh + r, sl = r % PF;
                    float h[NS];
#pragma unroll
                    for (int n = 0; n < NS; n += 4) {
                        h[n] = hs[sl][n / 4].x; h[n + 1] = hs[sl][n / 4].y; h[n + 2] = hs[sl][n / 4].z; h[n + 3] = hs[sl][n / 4].w;
                    }
                    const float y = scan_update<NS, R>(sF + row * FW, dtv[r], av, Dc, xv[sl], zs[sl], h);
#pragma unroll
                    for (int n = 0; n < NS; n += 4) buf_st4(sr, h_off(row, n), f32x4{h[n], h[n + 1], h[n + 2], h[n + 3]});
                    scr_st1(rscr, (uint32_t)(row * 2 * DI + DI + cq) * 4, y);
                }
            }
        }
        __syncthreads();  // every y written, dbc no longer read
        // ---- out_proj: y [ROWS][1024] in two K halves of 512 staged (split) through the operand buffer; wave w
        //      owns outputs 16 (NFO w + j) .. (j < NFO), both M fragments, accumulating the 32 K steps in order.
        //      Its blocks stream through a ring of one K step (NFO blocks) in use order.
        floatx4 acco[NFO][MF];
#pragma unroll
        for (int j = 0; j < NFO; ++j)
#pragma unroll
            for (int m = 0; m < MF; ++m) acco[j][m] = floatx4{0.f, 0.f, 0.f, 0.f};
        {
            LAYER_VARS
            const gptr<uint16_t> wop = G(w.out_p);
            u32x4 oh[DB], ol[DB];
            // block i of half hf: fragment NFO w + i % NFO, K step 16 hf + i / NFO
            auto issue_o = [&](int hf, int i) {
                const gptr<uint16_t> p =
                    wop + ((int64_t)(NFO * wave + (i % NFO)) * (DI / 32) + 16 * hf + i / NFO) * BLK + lane * 8;
                oh[i % DB] = ldg16(p);
                ol[i % DB] = wblk_lo<NT>(p, oh[i % DB]);
            };
#pragma unroll
            for (int i = 0; i < DB; ++i) issue_o(0, i);
#pragma unroll 1
            for (int hf = 0; hf < 2; ++hf) {
                {
                    SCR_VARS
                    // ROWS x 512 columns: thread t stages row t / 16, columns 32 (t % 16) + 4 e .. (e < 8)
                    const int r = tid >> 4, k0 = 32 * (tid & 15);
                    u32x4 u[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) u[e] = scr_ld16(rscr, (uint32_t)(r * 2 * DI + DI + 512 * hf + k0 + 4 * e) * 4);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        uint2 hp, lp;
                        split4(__uint_as_float(u[e].x), __uint_as_float(u[e].y), __uint_as_float(u[e].z),
                               __uint_as_float(u[e].w), hp, lp);
                        const int o = a_off(r, k0 + 4 * e);
                        *reinterpret_cast<uint2*>(sAh + o) = hp;
                        *reinterpret_cast<uint2*>(sAl + o) = lp;
                    }
                }
                __syncthreads();
                {
                    LANE_VARS
                    const int hn = hf + 1 < 2 ? hf + 1 : hf;
#pragma unroll
                    for (int s = 0; s < 16; ++s) {
                        bf16x8 ah[MF], al[MF];
#pragma unroll
                        for (int m = 0; m < MF; ++m) {
                            const int o = a_off(16 * m + ar, 32 * s + kq);
                            ah[m] = *reinterpret_cast<const bf16x8*>(sAh + o);
                            al[m] = *reinterpret_cast<const bf16x8*>(sAl + o);
                        }
#pragma unroll
                        for (int j = 0; j < NFO; ++j) {
                            const int i = NFO * s + j;
#pragma unroll
                            for (int m = 0; m < MF; ++m)
                                acco[j][m] = mfma_split_step<NT>(acco[j][m], ah[m], al[m], __builtin_bit_cast(bf16x8, oh[i % DB]),
                                                                 __builtin_bit_cast(bf16x8, ol[i % DB]));
                            if (i + DB < 16 * NFO) issue_o(hf, i + DB);
                            else issue_o(hn, i + DB - 16 * NFO);
                            pin_loads();
                        }
                    }
                }
                __syncthreads();  // the next half (or mm) rewrites the operand buffer
            }
        }
        // ---- mm = out_proj + bias as fp32 [ROWS][D] in the operand buffer
        {
            LANE_VARS
            LAYER_VARS
#pragma unroll
            for (int j = 0; j < NFO; ++j) {
                const int col = 16 * (NFO * wave + j) + ar;
                const float bias = G(w.out_b)[col];
#pragma unroll
                for (int m = 0; m < MF; ++m)
#pragma unroll
                    for (int i = 0; i < 4; ++i) sF[(16 * m + m_of + i) * D + col] = epi_value<EPI_BIAS>(acco[j][m][i], bias);
            }
        }
        __syncthreads();
        // ---- LN2 of this wave's rows: all read before any split is written over the fp32 rows
        {
            LANE_VARS
            LAYER_VARS
            float vv[RPW][8];
#pragma unroll
            for (int q = 0; q < RPW; ++q) {
                const int r = RPW * wave + q;
                const float4 u0 = *reinterpret_cast<const float4*>(sF + r * D + l4);
                const float4 u1 = *reinterpret_cast<const float4*>(sF + r * D + 256 + l4);
                vv[q][0] = u0.x; vv[q][1] = u0.y; vv[q][2] = u0.z; vv[q][3] = u0.w;
                vv[q][4] = u1.x; vv[q][5] = u1.y; vv[q][6] = u1.z; vv[q][7] = u1.w;
            }
            const float4 w0 = ldg_f4(G(w.ln2_w) + l4), w1 = ldg_f4(G(w.ln2_w) + 256 + l4);
            const float4 c0 = ldg_f4(G(w.ln2_b) + l4), c1 = ldg_f4(G(w.ln2_b) + 256 + l4);
            const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
            const float bv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            __syncthreads();
#pragma unroll
            for (int q = 0; q < RPW; ++q) {
                const int r = RPW * wave + q;
                float mu, rs;
                ln_stats_row<2>(vv[q], mu, rs);
                float y[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) y[i] = ln_apply(vv[q][i], mu, rs, wv[i], bv[i]);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    uint2 hp, lp;
                    split4(y[4 * h], y[4 * h + 1], y[4 * h + 2], y[4 * h + 3], hp, lp);
                    const int o = a_off(r, 256 * h + l4);
                    *reinterpret_cast<uint2*>(sAh + o) = hp;
                    *reinterpret_cast<uint2*>(sAl + o) = lp;
                }
            }
        }
        __syncthreads();

        // ---- feed-forward in 16 chunks of 128 hidden units: FF1 (+bias, GELU) of the chunk as in in_proj, split into
        //      the chunk buffer; FF2 accumulates the chunk's 4 K steps (wave w owns outputs 16 (NFO w + j) .., both
        //      M fragments).  Two rings, each running on into the next chunk.
        floatx4 accf[NFO][MF];
#pragma unroll
        for (int j = 0; j < NFO; ++j)
#pragma unroll
            for (int m = 0; m < MF; ++m) accf[j][m] = floatx4{0.f, 0.f, 0.f, 0.f};
        {
            LAYER_VARS
            const gptr<uint16_t> w1p = G(w.ff1_p), w2p = G(w.ff2_p);
            u32x4 rh[DK][NFC], rl[DK][NFC];
            auto issue1 = [&](int c, int s) {
#pragma unroll
                for (int n = 0; n < NFC; ++n) {
                    const gptr<uint16_t> q = w1p + ((int64_t)(8 * c + NFC * wave + n) * KSD + s) * BLK + lane * 8;
                    rh[s % DK][n] = ldg16(q);
                    rl[s % DK][n] = wblk_lo<NT>(q, rh[s % DK][n]);
                }
            };
            u32x4 oh[DB], ol[DB];
            // block i of chunk c: fragment NFO w + i % NFO, K step 4 c + i / NFO (K = 2048: 64 steps)
            auto issue2 = [&](int c, int i) {
                const gptr<uint16_t> p =
                    w2p + ((int64_t)(NFO * wave + (i % NFO)) * (4 * D / 32) + 4 * c + i / NFO) * BLK + lane * 8;
                oh[i % DB] = ldg16(p);
                ol[i % DB] = wblk_lo<NT>(p, oh[i % DB]);
            };
#pragma unroll
            for (int s = 0; s < DK; ++s) issue1(0, s);
#pragma unroll
            for (int i = 0; i < DB; ++i) issue2(0, i);
            constexpr int NHC = 4 * D / CH;
#pragma unroll 1
            for (int c = 0; c < NHC; ++c) {
                LANE_VARS
                const int cn = c + 1 < NHC ? c + 1 : c;
                float4 bias[NFC];
#pragma unroll
                for (int n = 0; n < NFC; ++n) bias[n] = ldg_f4(G(w.ff1_b) + 16 * (8 * c + NFC * wave + n) + m_of);
                floatx4 acc[NFC][MF];
#pragma unroll
                for (int n = 0; n < NFC; ++n)
#pragma unroll
                    for (int m = 0; m < MF; ++m) acc[n][m] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < KSD; ++s) {
                    chunk_kstep<NT>(acc, sAh, sAl, s, ar, kq, rh[s % DK], rl[s % DK]);
                    if (s + DK < KSD) issue1(c, s + DK);
                    else issue1(cn, s + DK - KSD);
                    pin_loads();
                }
#pragma unroll
                for (int n = 0; n < NFC; ++n) {
                    const float bb[4] = {bias[n].x, bias[n].y, bias[n].z, bias[n].w};
#pragma unroll
                    for (int m = 0; m < MF; ++m) {
                        float g[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i) g[i] = epi_value<EPI_GELU>(acc[n][m][i], bb[i]);
                        uint2 hp, lp;
                        split4(g[0], g[1], g[2], g[3], hp, lp);
                        const int oc = c_off(16 * m + ar, 16 * (NFC * wave + n) + m_of);
                        *reinterpret_cast<uint2*>(sCh + oc) = hp;
                        *reinterpret_cast<uint2*>(sCl + oc) = lp;
                    }
                }
                __syncthreads();
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    bf16x8 ah[MF], al[MF];
#pragma unroll
                    for (int m = 0; m < MF; ++m) {
                        const int o = c_off(16 * m + ar, 32 * s + kq);
                        ah[m] = *reinterpret_cast<const bf16x8*>(sCh + o);
                        al[m] = *reinterpret_cast<const bf16x8*>(sCl + o);
                    }
#pragma unroll
                    for (int j = 0; j < NFO; ++j) {
                        const int i = NFO * s + j;
#pragma unroll
                        for (int m = 0; m < MF; ++m)
                            accf[j][m] = mfma_split_step<NT>(accf[j][m], ah[m], al[m], __builtin_bit_cast(bf16x8, oh[i % DB]),
                                                             __builtin_bit_cast(bf16x8, ol[i % DB]));
                        if (i + DB < 4 * NFO) issue2(c, i + DB);
                        else issue2(cn, i + DB - 4 * NFO);
                        pin_loads();
                    }
                }
                __syncthreads();
            }
        }
        // ---- residual: x <- x + (FF2 + bias), element by element in LDS (each element has one owner thread)
        {
            LANE_VARS
            LAYER_VARS
#pragma unroll
            for (int j = 0; j < NFO; ++j) {
                const int col = 16 * (NFO * wave + j) + ar;
                const float bias = G(w.ff2_b)[col];
#pragma unroll
                for (int m = 0; m < MF; ++m)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        float& x = sRes[(16 * m + m_of + i) * LRS + col];
                        x = x + epi_value<EPI_RESID>(accf[j][m][i], bias);
                    }
            }
        }
        __syncthreads();
    }

    // ---- head: Linear -> ReLU -> Linear (model.py:95, 101), hidden layer in 4 chunks of 128
    {
        LANE_VARS
        u32x4 ru[RPW][2];
#pragma unroll
        for (int q = 0; q < RPW; ++q)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                ru[q][h] = *reinterpret_cast<const u32x4*>(sRes + (RPW * wave + q) * LRS + 256 * h + l4);
#pragma unroll
        for (int q = 0; q < RPW; ++q)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const u32x4 u = ru[q][h];
                uint2 hp, lp;
                split4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w), hp, lp);
                const int o = a_off(RPW * wave + q, 256 * h + l4);
                *reinterpret_cast<uint2*>(sAh + o) = hp;
                *reinterpret_cast<uint2*>(sAl + o) = lp;
            }
    }
    __syncthreads();
    floatx4 acch[NFH][MF];
#pragma unroll
    for (int j = 0; j < NFH; ++j)
#pragma unroll
        for (int m = 0; m < MF; ++m) acch[j][m] = floatx4{0.f, 0.f, 0.f, 0.f};
    {
        const gptr<uint16_t> w1p = G(a.h1_p), w2p = G(a.h2_p);
#pragma unroll 1
        for (int c = 0; c < D / CH; ++c) {
            LANE_VARS
            floatx4 acc[NFC][MF];
#pragma unroll
            for (int n = 0; n < NFC; ++n)
#pragma unroll
                for (int m = 0; m < MF; ++m) acc[n][m] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
            for (int s = 0; s < KSD; ++s) {
                u32x4 bh[NFC], bl[NFC];
#pragma unroll
                for (int n = 0; n < NFC; ++n) {
                    const gptr<uint16_t> p = w1p + ((int64_t)(8 * c + NFC * wave + n) * KSD + s) * BLK + lane * 8;
                    bh[n] = ldg16(p);
                    bl[n] = wblk_lo<NT>(p, bh[n]);
                }
                chunk_kstep<NT>(acc, sAh, sAl, s, ar, kq, bh, bl);
            }
#pragma unroll
            for (int n = 0; n < NFC; ++n) {
                const float4 bias = ldg_f4(G(a.h1_b) + 16 * (8 * c + NFC * wave + n) + m_of);
                const float bb[4] = {bias.x, bias.y, bias.z, bias.w};
#pragma unroll
                for (int m = 0; m < MF; ++m) {
                    float g[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) g[i] = epi_value<EPI_RELU>(acc[n][m][i], bb[i]);
                    uint2 hp, lp;
                    split4(g[0], g[1], g[2], g[3], hp, lp);
                    const int oc = c_off(16 * m + ar, 16 * (NFC * wave + n) + m_of);
                    *reinterpret_cast<uint2*>(sCh + oc) = hp;
                    *reinterpret_cast<uint2*>(sCl + oc) = lp;
                }
            }
            __syncthreads();
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                bf16x8 ah[MF], al[MF];
#pragma unroll
                for (int m = 0; m < MF; ++m) {
                    const int o = c_off(16 * m + ar, 32 * s + kq);
                    ah[m] = *reinterpret_cast<const bf16x8*>(sCh + o);
                    al[m] = *reinterpret_cast<const bf16x8*>(sCl + o);
                }
#pragma unroll
                for (int j = 0; j < NFH; ++j) {
                    const gptr<uint16_t> p = w2p + ((int64_t)(NFH * wave + j) * KSD + 4 * c + s) * BLK + lane * 8;
                    const u32x4 bh = ldg16(p), bl = wblk_lo<NT>(p, bh);
#pragma unroll
                    for (int m = 0; m < MF; ++m)
                        acch[j][m] = mfma_split_step<NT>(acch[j][m], ah[m], al[m], __builtin_bit_cast(bf16x8, bh),
                                                         __builtin_bit_cast(bf16x8, bl));
                }
            }
            __syncthreads();
        }
    }
    // logits [ROWS][LLOG] fp32 in the operand buffer
    {
        LANE_VARS
#pragma unroll
        for (int j = 0; j < NFH; ++j) {
            const int col = 16 * (NFH * wave + j) + ar;
            const float bias = G(a.h2_b)[col];
#pragma unroll
            for (int m = 0; m < MF; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i) sF[(16 * m + m_of + i) * LLOG + col] = epi_value<EPI_BIAS>(acch[j][m][i], bias);
        }
    }
    __syncthreads();
    if (a.logits) {
        for (int i = tid; i < ROWS * VV; i += NTHR) {
            const int r = i / VV, n = i % VV;
            if (r < nb) a.logits[(b0 + r) * VV + n] = sF[r * LLOG + n];
        }
    }
    if (a.decode) {
#pragma unroll 1
        for (int q = 0; q < RPW; ++q) {
            const int r = RPW * wave + q;
            if (r >= nb) continue;
            const int64_t b = b0 + r;
            if (t >= a.lens[b]) continue;
            DecState st = a.dec[b];
            const LaneWords w = lane_words(a.payload, a.payload_words, a.off, a.nwords, b);
            const int s = decode_row(sF + r * LLOG, VV, lane, st, w.p, w.n);
            tokv = lane == q ? s : tokv;
            if (lane == 0) {
                a.dec[b] = st;
                a.out[b * a.out_stride + t] = (uint8_t)s;
            }
        }
    }
    __syncthreads();  // the next step rewrites the operand buffer
    p0m3 = p0m3 == 2 ? 0 : p0m3 + 1;
    }
    if (a0.decode) {
#pragma unroll
        for (int q = 0; q < RPW; ++q) {
            const int r = RPW * wave + q;
            const int tq = __builtin_amdgcn_readlane(tokv, q);
            if (r < nb && lane == 0) a0.tokens_out[b0 + r] = tq;
        }
    }
}

}  // namespace

bool fused_step512_supported(int d_model, int d_state, int dt_rank, int d_conv, int vocab) {
    return d_model == D && d_state == NS && dt_rank == R && d_conv == 4 && vocab == VV;
}

hipError_t launch_fused_step512(const FusedArgs& a, int nt, hipStream_t s) {
    const dim3 grid((unsigned)((a.B + ROWS - 1) / ROWS));
    if (nt == 3) hipLaunchKernelGGL((k_fused_step512<3>), grid, dim3(NTHR), 0, s, a);
    else hipLaunchKernelGGL((k_fused_step512<2>), grid, dim3(NTHR), 0, s, a);
    return hipGetLastError();
}

}  // namespace boa
