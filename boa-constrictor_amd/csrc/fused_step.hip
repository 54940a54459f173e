// Fused decompress steps: the whole model for 16 chunk lanes per workgroup, many positions per launch:
// embedding -> L x (LN1, in_proj, conv, x_proj, dt_proj + selective scan, out_proj, LN2, FF1 + GELU,
// FF2 + residual) -> head (Linear-ReLU-Linear) -> quantiser + range decoder -> next byte, which is the
// next step's input without leaving the workgroup.
//
// Reference: the per-step loop of codec.py:211-323 (decompress_GPU: model.step on the batch of streams,
// softmax, Q2 table, coder.decode_step) and of portability_solved_cpp/boa.cpp:556-569 (step_batch +
// gpu_rc_decode_fused_step_batch), done here without leaving the chip between layers.
//
// Design (gfx950): 512 threads (8 waves) own 16 lanes = the M of one v_mfma_f32_16x16x32_bf16 fragment.
// Activations stay in LDS for the whole step (141 KB: residual stream, split-bf16 GEMM operand, xz / FF
// hidden, x_proj partials and dt|B|C rows); GEMM weights stream from L2 in fragment-packed blocks (one
// coalesced 16-byte load per lane per block); the only HBM traffic is the recurrent state (SSM state and the
// conv history ring) and the step's inputs and outputs.  Lanes are independent, so a workgroup runs its
// steps without any grid-wide synchronisation (workgroup classes can start at offsets, stagger_us, off by
// default).  GEMM phases: wave w computes output fragments w, w + 8, ...; each
// output accumulates 32-wide K steps in ascending order, lo*hi, hi*lo, hi*hi per step, exactly as the tiled
// split-precision GEMM does, and every elementwise phase calls the same device function as the tiled
// path (model_dev.h).  The logits of a lane are therefore bit-identical to those the compress path
// computes for the same position, which the decoder depends on.
// NT = 1 is the fp32 precision mode: the GEMM operands are fp32 in LDS (the same regions, rows 4 elements
// shorter) and every output accumulates 16-wide K groups of four v_mfma_f32_16x16x4_f32 in ascending order,
// lane l supplying k = 16 g + 4 (l / 16) + j to the j-th, exactly as the tiled fp32 GEMM (k_gemm) does; x_proj
// is the same K-block fold as in the split modes (each 64-channel partial from zero in the wave that produced
// those channels, then P_0 + P_1 + ...), as every fp32 path computes it.
#include "model_dev.h"
#include "model_internal.h"

namespace boa {

namespace {

constexpr int FD = 256;             // d_model
constexpr int FDI = 512;            // d_inner
constexpr int FNS = 16;             // d_state
constexpr int FR = 16;              // dt_rank
constexpr int FW = FR + 2 * FNS;    // x_proj width (dt | B | C)
constexpr int ROWS = 16;            // lanes per workgroup

constexpr int LRES = FD + 4;        // fp32 rows of 256 (+4: conflict-free fragment-order writes)
constexpr int LA = FDI + 8;         // split operand rows, K <= 512 (bf16 elements)
constexpr int LXZ = 2 * FDI + 4;    // in_proj output rows (fp32)
constexpr int LH = 4 * FD + 8;      // FF hidden split rows, K = 1024 (bf16 elements)
constexpr int LH1 = FD + 8;         // head hidden split rows, K = 256
// fp32 operand rows (NT = 1) in the same regions: 4 elements shorter, 4 mod 64 words, so that 16-row float4
// reads are free of bank conflicts
constexpr int ld32(int LD) { return LD - 4; }

constexpr int SZ_RES = ROWS * LRES * 4;
constexpr int SZ_A = 2 * ROWS * LA * 2;
constexpr int SZ_X = (ROWS * LXZ * 4 > 2 * ROWS * LH * 2) ? ROWS * LXZ * 4 : 2 * ROWS * LH * 2;
constexpr int SZ_DBC = (FDI / XPROJ_KB) * ROWS * FW * 4;  // x_proj partials; dbc in place of the first
constexpr int OFF_RES = 0;
constexpr int OFF_A = OFF_RES + SZ_RES;
constexpr int OFF_X = OFF_A + SZ_A;
constexpr int OFF_DBC = OFF_X + SZ_X;
constexpr int LDS_BYTES = OFF_DBC + SZ_DBC;
static_assert(LDS_BYTES <= 160 * 1024, "fused step LDS budget");
static_assert(OFF_A % 16 == 0 && OFF_X % 16 == 0 && OFF_DBC % 16 == 0, "LDS alignment");
static_assert(ROWS * LRES * 4 <= SZ_A, "logits tile must fit the operand region");

// C[16][16 nfrag] = A[16][K] (split bf16 in LDS, row stride lda) x W^T (fragment-packed), for this wave's
// fragments f = rot(f0 + wave + NWAVE j) (j < FPW, f0 + wave + NWAVE j < nfrag), rot(f) = (f + rot) mod nfrag.  B
// blocks of D - 1 K steps ahead are in flight (a register ring) while the current step is multiplied: one
// workgroup per CU streams every weight of the layer from L2, so latency bounds a shallow pipeline.  The
// rotation (per workgroup) spreads the workgroups of an XCD over different weight blocks at any moment
// instead of all reading the same L2 lines; it does not change any output (each output fragment still
// accumulates its K steps in ascending order).  Output column of acc[j]: 16 * frag_of(...) + lane % 16.
template <int NWAVE>
__device__ __forceinline__ int frag_of(int f0, int wave, int j, int nfrag, int rot) {
    const int f = f0 + wave + NWAVE * j + rot;
    return f >= nfrag ? f - nfrag : f;
}

// The fp32 form (NT = 1): A fp32 in LDS (row stride lda), W from fp32 fragment-packed blocks (block (f, g): lane
// l holds W[16 f + l % 16][16 g + 4 (l / 16) + j], j < 4, one 16-byte load).  Each output accumulates its 16-K
// groups in ascending order, the j-th MFMA of group g taking k = 16 g + 4 (l / 16) + j from lane l, which is
// k_gemm's order.  RD groups are in flight through a register ring; the loop runs over passes of RD groups so
// that every ring slot is fixed per unrolled position, and the last prefetches are clamped to the last group
// (reloads, unused) instead of sitting under a branch.  Each group's weight loads and the next group's A
// fragment are issued together and pinned there (left to itself the scheduler sinks the loads to their uses).
// Within a group the MFMAs go round the fragments (x of every fragment, then y, ...); each fragment's own
// sequence is unchanged.
// CHECK: whether some of this wave's fragments may lie past nfrag.  When the caller's shape rules that out
// (nfrag a multiple of FPW * NWAVE, f0 a multiple of it too) there is no per-fragment condition at all: a load or
// MFMA under a branch costs an exec-mask round trip, and an accumulator merged after a branch costs a wait for
// the MFMA result and register copies, in every group (fp32 step 0.90 -> 0.86 ms with the other changes here).
template <int NWAVE, int FPW, int K, int RD, bool CHECK>
__device__ __forceinline__ void mgemm_f32(const float* A, int lda, const float* __restrict__ Wp, int f0, int nfrag,
                                          int wave, int lane, int rot, floatx4 (&acc)[FPW]) {
    constexpr int S = K / 16;
    static_assert(S % RD == 0, "whole passes of the register ring");
    const int kq = 4 * (lane >> 4), ar = lane & 15;
    const int fw = f0 + wave;
    auto valid = [&](int j) { return !CHECK || fw + NWAVE * j < nfrag; };
#pragma unroll
    for (int j = 0; j < FPW; ++j) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    float4 bw[RD][FPW];
    // Weight loads through a buffer descriptor: a fragment's lane offset sits in the vector operand (formed once per
    // pass), the group's offset (g KB) in the scalar one, so a load costs no vector address arithmetic.  (With
    // 64-bit global addresses, two VALU adds per load competed with the MFMAs for issue: an isolated in_proj phase
    // took 18.8-20 us against 15.1-15.3 us with this form.)
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(Wp, (uint32_t)nfrag * S * 1024u);
    uint32_t voff[FPW];
#pragma unroll
    for (int j = 0; j < FPW; ++j) voff[j] = (uint32_t)(frag_of<NWAVE>(f0, wave, j, nfrag, rot) * S * 1024 + lane * 16);
    auto load = [&](int g, int slot) {
#pragma unroll
        for (int j = 0; j < FPW; ++j) {
            if (valid(j)) {
                const f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, voff[j], g * 1024, 0));
                bw[slot][j] = make_float4(v.x, v.y, v.z, v.w);
            }
        }
    };
    const float* Ar = A + ar * lda + kq;
#pragma unroll
    for (int i = 0; i < RD - 1; ++i) load(i, i);
    float4 a = *reinterpret_cast<const float4*>(Ar);
#pragma unroll 1
    for (int g0 = 0; g0 < S; g0 += RD) {
#pragma unroll
        for (int i = 0; i < RD; ++i) {
            const int gn = g0 + i + RD - 1;
            load(gn < S ? gn : S - 1, (i + RD - 1) % RD);
            // the next group's A fragment (the last group re-reads its own), read one group ahead
            const int ga = g0 + i + 1 < S ? g0 + i + 1 : S - 1;
            const float4 an = *reinterpret_cast<const float4*>(Ar + 16 * ga);
            pin_loads();  // issued here, ahead of their use (the scheduler would sink them to it)
            const float av[4] = {a.x, a.y, a.z, a.w};
            a = an;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
#pragma unroll
                for (int j = 0; j < FPW; ++j) {
                    if (valid(j)) {
                        const float4 b = bw[i][j];
                        const float bv[4] = {b.x, b.y, b.z, b.w};
                        acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], bv[e], acc[j], 0, 0, 0);
                    }
                }
            }
        }
    }
}

// D: K steps in flight in the split forms; RDF: 16-K groups in flight in the fp32 form.
template <int NT, int NWAVE, int FPW, int K, int D, bool CHECK = true, int RDF = 4>
__device__ __forceinline__ void mgemm(const uint16_t* sAh, const uint16_t* sAl, int lda,
                                      const uint16_t* __restrict__ Wp, int f0, int nfrag, int wave, int lane,
                                      int rot, floatx4 (&acc)[FPW]) {
    if constexpr (NT == 1) {
        mgemm_f32<NWAVE, FPW, K, RDF, CHECK>(reinterpret_cast<const float*>(sAh), ld32(lda),
                                           reinterpret_cast<const float*>(Wp), f0, nfrag, wave, lane, rot, acc);
        return;
    }
    constexpr int BLK = (NT == 3) ? 1024 : 512;
    constexpr int S = K / 32;
    const int kq = 8 * (lane >> 4), ar = lane & 15;
    const int fw = f0 + wave;
    // The split forms keep the per-fragment condition whatever CHECK says: without it the compiler hoists the
    // fully unrolled loop's loads together and the ring no longer spaces them (FF1 measured 40% slower).
    auto valid = [&](int j) { return fw + NWAVE * j < nfrag; };
#pragma unroll
    for (int j = 0; j < FPW; ++j) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    uint4 bh[D][FPW], bl[D][FPW];
    auto load = [&](int s, int slot) {
#pragma unroll
        for (int j = 0; j < FPW; ++j) {
            if (valid(j)) {
                const int f = frag_of<NWAVE>(f0, wave, j, nfrag, rot);
                const gptr<uint16_t> p = G(Wp) + ((int64_t)f * S + s) * BLK + lane * 8;
                bh[slot][j] = __builtin_bit_cast(uint4, ldg16(p));
                if constexpr (NT == 3) bl[slot][j] = __builtin_bit_cast(uint4, ldg16(p + 512));
            }
        }
    };
#pragma unroll
    for (int s = 0; s < D - 1; ++s)
        if (s < S) load(s, s);
#pragma unroll
    for (int s = 0; s < S; ++s) {
        if (s + D - 1 < S) load(s + D - 1, (s + D - 1) % D);
        const bf16x8 ah = *reinterpret_cast<const bf16x8*>(sAh + ar * lda + 32 * s + kq);
        const bf16x8 al = *reinterpret_cast<const bf16x8*>(sAl + ar * lda + 32 * s + kq);
#pragma unroll
        for (int j = 0; j < FPW; ++j) {
            if (valid(j)) {
                const bf16x8 h = __builtin_bit_cast(bf16x8, bh[s % D][j]);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, h, acc[j], 0, 0, 0);
                if constexpr (NT == 3)
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, __builtin_bit_cast(bf16x8, bl[s % D][j]),
                                                                     acc[j], 0, 0, 0);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, h, acc[j], 0, 0, 0);
            }
        }
    }
}

__device__ __forceinline__ void put_split(uint16_t* h, uint16_t* l, int idx, float v) {
    uint32_t hi, lo;
    split2(v, hi, lo);
    h[idx] = (uint16_t)hi;
    l[idx] = (uint16_t)lo;
}

// GEMM operand regions: split bf16 rows of LD elements (hi array, then lo array at h + ROWS * LD), or with
// NT = 1 fp32 rows of ld32(LD) elements over the same bytes.
template <int NT, int LD>
__device__ __forceinline__ void store_op(uint16_t* h, int r, int c, float v) {
    if constexpr (NT == 1) reinterpret_cast<float*>(h)[r * ld32(LD) + c] = v;
    else put_split(h, h + ROWS * LD, r * LD + c, v);
}

// LayerNorm of rows RPW*wave .. RPW*wave + RPW-1 of src (fp32, stride LRES) into the split operand (stride LA).
// wv, bv: this lane's 4 weights and biases, loaded by the caller ahead of the barrier before the LN phase, so
// their L2 round trip (behind the pointer load from the layer table) overlaps the previous phase's tail.
template <int NT, int RPW>
__device__ __forceinline__ void ln_rows(const float* src, float4 wv, float4 bv, uint16_t* sAh, uint16_t* sAl, int wave,
                                       int lane) {
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
        const int r = RPW * wave + q;
        const float4 x4 = *reinterpret_cast<const float4*>(src + r * LRES + 4 * lane);
        const float v[4] = {x4.x, x4.y, x4.z, x4.w};
        float mu, rs;
        ln_stats_row<1>(v, mu, rs);
        const float y[4] = {ln_apply(v[0], mu, rs, wv.x, bv.x), ln_apply(v[1], mu, rs, wv.y, bv.y),
                            ln_apply(v[2], mu, rs, wv.z, bv.z), ln_apply(v[3], mu, rs, wv.w, bv.w)};
        if constexpr (NT == 1) {
            *reinterpret_cast<float4*>(reinterpret_cast<float*>(sAh) + r * ld32(LA) + 4 * lane) =
                make_float4(y[0], y[1], y[2], y[3]);
        } else {
            uint2 hp, lp;
            split4(y[0], y[1], y[2], y[3], hp, lp);
            *reinterpret_cast<uint2*>(sAh + r * LA + 4 * lane) = hp;
            *reinterpret_cast<uint2*>(sAl + r * LA + 4 * lane) = lp;
        }
    }
}

typedef __attribute__((address_space(4))) const FusedArgs KArgs;

// 512 threads: 8 waves (2 per SIMD); wave w owns channels 64w .. 64w + 63 in the conv and scan phases, which
// is x_proj's K block w (XPROJ_KB).
template <int NT, int NTHR>
__global__ void __launch_bounds__(NTHR) k_fused_step(FusedArgs a) {
    constexpr int NWAVE = NTHR / 64;
    constexpr int RPW = ROWS / NWAVE;               // rows per wave (LN, decode)
    // fragments per wave and pass, N = 1024 GEMMs (in_proj, FF1): 4 in the split forms (two passes); 8 in the fp32
    // form (one pass), with 2 groups of 16 K in flight (the widest fragment set with the buffer-loaded weights measured
    // best: 0.79 ms per step against 0.80 with 2 fragments and 16 groups in flight, 0.82 with 4 and 4)
    constexpr int FPW_B = NT == 1 ? 8 : 4;
    constexpr int D_B = 3;         // K steps in flight, N = 1024 GEMMs
    constexpr int FPW_S = 16 / NWAVE;               // fragments per wave, N = 256 GEMMs
    constexpr int D_S = 6;         // K steps in flight, N = 256 GEMMs
    // lane 0's SSM state is loaded before the x_proj fold in the fp32 form (with the per-channel scan parameters,
    // which every form loads there)
    constexpr bool HOIST_FIRST = NT == 1;
    static_assert(NTHR == 512 && NTHR == FDI && NWAVE * XPROJ_KB == FDI, "fused step block size: one thread per channel");
    // every GEMM below but x_proj and head2 covers its fragments exactly (mgemm's CHECK = false)
    static_assert((2 * FDI / 16) % (FPW_B * NWAVE) == 0 && (4 * FD / 16) % (FPW_B * NWAVE) == 0 &&
                  (FD / 16) % (FPW_S * NWAVE) == 0, "whole passes of fragments");
    __shared__ __attribute__((aligned(16))) unsigned char lds[LDS_BYTES];
    float* sRes = reinterpret_cast<float*>(lds + OFF_RES);
    uint16_t* sAh = reinterpret_cast<uint16_t*>(lds + OFF_A);
    uint16_t* sAl = sAh + ROWS * LA;
    float* sX = reinterpret_cast<float*>(lds + OFF_X);
    uint16_t* sHh = reinterpret_cast<uint16_t*>(lds + OFF_X);
    uint16_t* sHl = sHh + ROWS * LH;
    float* sPart = reinterpret_cast<float*>(lds + OFF_DBC);  // x_proj partials [8][ROWS][FW]
    float* sDbc = sPart;                                      // their sum, in place of the first
    float* sLog = reinterpret_cast<float*>(lds + OFF_A);  // head output (operand region is free by then)

    __shared__ int sTok[ROWS];
    __shared__ int sMaxLen;

    const int tid = threadIdx.x, lane = tid & 63;
    // uniform: a scalar register in the fp32 form (the split forms measured slower with it, 0.59 -> 0.67 ms per
    // step together with the per-layer lane copies below, and keep the plain form)
    const int wave = NT == 1 ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6;
    const int64_t b0 = (int64_t)blockIdx.x * ROWS;
    const int nb = (int)((a.B - b0) < ROWS ? (a.B - b0) : ROWS);  // valid lanes of this workgroup
    const int V = a.V;
    if (tid < ROWS) sTok[tid] = tid < nb ? a.tokens_in[b0 + tid] : 0;
    if (tid == 0) {
        int ml = 0;
        if (a.decode)
            for (int r = 0; r < nb; ++r) ml = a.lens[b0 + r] > ml ? a.lens[b0 + r] : ml;
        sMaxLen = ml;
        // start offset of this workgroup's class: classes are sets of XCDs (workgroup i runs on XCD i mod 8),
        // which do not share an L2, so a following class does not catch up on the leaders' L2 hits
        if (a.stagger_us > 0 && a.stagger_classes > 1) {
            const int cls = (int)(blockIdx.x & 7) * a.stagger_classes / 8;
            const uint64_t until = wall_clock64() + (uint64_t)(cls * a.stagger_us) * 100u;
            while (wall_clock64() < until) __builtin_amdgcn_s_sleep(8);
        }
    }
    __syncthreads();
    // (a lane's first output row in a fragment, m_of, and its column, n_of, are formed per layer and for the head)

    int p0m3 = a.p0m3;
#pragma unroll 1
    for (int step = 0; step < a.nsteps; ++step) {
    const int t = a.t + step;
    // Per-workgroup values are re-derived in every step from an opaque copy of the block index, so that
    // the compiler does not keep dozens of loop-invariant lane addresses live across the whole step.
    // The kernel arguments are read again through an opaque pointer to the kernarg segment for the
    // same reason (otherwise every field stays in SGPRs across the loop and spills).
    int bid = (int)blockIdx.x;
    __asm__ volatile("" : "+s"(bid));
    auto kp = (__attribute__((address_space(4))) const char*)__builtin_amdgcn_kernarg_segment_ptr();
    __asm__ volatile("" : "+s"(kp));
    KArgs& a = *reinterpret_cast<KArgs*>(kp);
    const int64_t b0 = (int64_t)bid * ROWS;
    // fragment rotations: consecutive workgroups of an XCD (blockIdx / 8) start on different weight blocks
    const int rot64 = ((bid >> 3) & 7) * 8, rot16 = (bid >> 3) & 15;
    if (a.decode && t >= sMaxLen) break;  // every lane of this workgroup is complete (uniform condition)
    // embedding (model.py:97): x = E[byte]
    for (int i = tid; i < ROWS * (FD / 4); i += NTHR) {
        const int r = i / (FD / 4), c4 = (i % (FD / 4)) * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < nb) {
            int tok = sTok[r];
            tok = tok < 0 ? 0 : (tok >= V ? V - 1 : tok);
            v = ldg_f4(G(a.emb) + (int64_t)tok * FD + c4);
        }
        *reinterpret_cast<float4*>(sRes + r * LRES + c4) = v;
    }
    float4 lnw = ldg_f4(G(layer_at(a.layers, 0).ln1_w) + 4 * lane), lnb = ldg_f4(G(layer_at(a.layers, 0).ln1_b) + 4 * lane);
    __syncthreads();

    const int s1 = p0m3 == 2 ? 0 : p0m3 + 1, s2 = p0m3 == 0 ? 2 : p0m3 - 1;

    for (int l = 0; l < a.L; ++l) {
        // Lane-derived values re-derived per layer from an opaque copy of the thread index, so that the compiler
        // does not form every phase's per-lane addresses once outside the layer loop and hold them (dozens of
        // registers) across all phases, which leaves the GEMM phases too few registers for their weight rings.
        int tid_o = (int)threadIdx.x;
        if constexpr (NT == 1) __asm__ volatile("" : "+v"(tid_o));
        const int tid = tid_o, lane = tid_o & 63;
        const int m_of = 4 * (lane >> 4), n_of = lane & 15;
        CFusedLayer& w = layer_at(a.layers, l);
        // ---- LN1 -> split operand
        ln_rows<NT, RPW>(sRes, lnw, lnb, sAh, sAl, wave, lane);
        __syncthreads();
        // ---- in_proj (+bias) -> xz fp32
#pragma unroll 1
        for (int f0 = 0; f0 < 2 * FDI / 16; f0 += FPW_B * NWAVE) {
            floatx4 acc[FPW_B];
            float bias_j[FPW_B];  // loaded ahead of the weight ring (in-order wait counter)
#pragma unroll
            for (int j = 0; j < FPW_B; ++j) bias_j[j] = G(w.in_b)[16 * frag_of<NWAVE>(f0, wave, j, 2 * FDI / 16, rot64) + n_of];
            mgemm<NT, NWAVE, FPW_B, FD, D_B, false, 2>(sAh, sAl, LA, w.in_p, f0, 2 * FDI / 16, wave, lane, rot64, acc);
#pragma unroll
            for (int j = 0; j < FPW_B; ++j) {
                const int n = 16 * frag_of<NWAVE>(f0, wave, j, 2 * FDI / 16, rot64) + n_of;
                const float bias = bias_j[j];
#pragma unroll
                for (int r = 0; r < 4; ++r) sX[(m_of + r) * LXZ + n] = epi_value<EPI_BIAS>(acc[j][r], bias);
            }
        }
        __syncthreads();
        // ---- conv + SiLU (thread = channel): xs fp32 in place of x, split operand, history ring; then this
        //      wavefront's x_proj partial P_wave over the 64 channels it has just produced (XPROJ_KB)
        {
            // x_proj weight blocks of this wave's K block, issued first (they do not depend on the step).  fp32
            // form: blocks (f, 4 wave + g), g < 4, of the fp32 fragment-packed matrix, two per 32-wide K step (in
            // the registers the split parts use)
            constexpr int XS = FDI / 32, XF = FW / 16, XBLK = (NT == 3) ? 1024 : 512;
            uint4 xwh[XF][2], xwl[XF][2];
            if constexpr (NT == 1) {
                const gptr<float> xp = G(reinterpret_cast<const float*>(w.x_p));
#pragma unroll
                for (int f = 0; f < XF; ++f)
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        const int g = 4 * wave + 2 * s;
                        xwh[f][s] = __builtin_bit_cast(uint4, ldg16(xp + ((int64_t)f * (FDI / 16) + g) * 256 + lane * 4));
                        xwl[f][s] = __builtin_bit_cast(uint4, ldg16(xp + ((int64_t)f * (FDI / 16) + g + 1) * 256 + lane * 4));
                    }
            } else {
#pragma unroll
                for (int f = 0; f < XF; ++f)
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        const gptr<uint16_t> p = G(w.x_p) + ((int64_t)f * XS + 2 * wave + s) * XBLK + lane * 8;
                        xwh[f][s] = __builtin_bit_cast(uint4, ldg16(p));
                        xwl[f][s] = xwh[f][s];
                        if constexpr (NT == 3) xwl[f][s] = __builtin_bit_cast(uint4, ldg16(p + 512));
                    }
            }
            const int c = tid;
            const float4 cw = ldg_f4(G(w.conv_w) + 4 * c);
            const float cb = G(w.conv_b)[c];
            // history ring of this workgroup's valid lanes [b0, b0 + nb): rows past the last lane read 0 and
            // are not written (buffer range check), so no access is under a branch
            const __amdgpu_buffer_rsrc_t hr3 =
                buf_rsrc(a.hist + ((int64_t)l * a.max_lanes + b0) * 3 * FDI, (uint32_t)nb * 3 * FDI * 4);
            // Per-lane offsets are formed inside each unrolled iteration from an opaque copy of the channel
            // index: precomputed for all lanes at once they would hold dozens of registers across the layer
            // loop, which spill, and every reload of a spilled offset (a vector memory load) waits for all the
            // state loads issued before it.
            float h0[ROWS], h1[ROWS], h2[ROWS];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                int cq = c;
                __asm__ volatile("" : "+v"(cq));
                const uint32_t o = (uint32_t)(r * 3 * FDI + cq) * 4;
                h0[r] = buf_ld1(hr3, o + p0m3 * FDI * 4);
                h1[r] = buf_ld1(hr3, o + s1 * FDI * 4);
                h2[r] = buf_ld1(hr3, o + s2 * FDI * 4);
            }
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                int cq = c;
                __asm__ volatile("" : "+v"(cq));
                const float x = sX[r * LXZ + cq];
                const float y = conv_point(cw, cb, h0[r], h1[r], h2[r], x);
                sX[r * LXZ + cq] = y;
                store_op<NT, LA>(sAh, r, cq, y);
                buf_st1(hr3, (uint32_t)(r * 3 * FDI + p0m3 * FDI + cq) * 4, x);
            }
            // the partial reads only values this wavefront wrote (channels 64 wave .. 64 wave + 63 of every row);
            // LDS operations of one wavefront complete in order
            {
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const int ar = lane & 15;
                floatx4 part[XF];
#pragma unroll
                for (int f = 0; f < XF; ++f) part[f] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    bf16x8 ah, al;
                    if constexpr (NT == 1) {
                        // fp32 rows: lane l's 4 values of groups 4 wave + 2 s and + 1 (k = 16 g + 4 (l / 16) + j)
                        const float* r32 = reinterpret_cast<const float*>(sAh) + ar * ld32(LA) + XPROJ_KB * wave +
                                           32 * s + 4 * (lane >> 4);
                        ah = __builtin_bit_cast(bf16x8, *reinterpret_cast<const float4*>(r32));
                        al = __builtin_bit_cast(bf16x8, *reinterpret_cast<const float4*>(r32 + 16));
                    } else {
                        const int k0 = XPROJ_KB * wave + 32 * s, kq = 8 * (lane >> 4);
                        ah = *reinterpret_cast<const bf16x8*>(sAh + ar * LA + k0 + kq);
                        al = *reinterpret_cast<const bf16x8*>(sAl + ar * LA + k0 + kq);
                    }
#pragma unroll
                    for (int f = 0; f < XF; ++f)
                        part[f] = mfma_split_step<NT>(part[f], ah, al, __builtin_bit_cast(bf16x8, xwh[f][s]),
                                                      __builtin_bit_cast(bf16x8, xwl[f][s]));
                }
                float* pw = sPart + wave * (ROWS * FW);
#pragma unroll
                for (int f = 0; f < XF; ++f)
#pragma unroll
                    for (int r = 0; r < 4; ++r) pw[(m_of + r) * FW + 16 * f + n_of] = part[f][r];
            }
        }
        __syncthreads();
        // ---- the scan's operands that do not depend on x_proj, issued ahead of it (their memory latency then
        //      overlaps x_proj): the channel's A row, dt_proj row, biases and lane 0's state (thread = channel)
        const int c = tid;
        float av[FNS], wr[FR];
        {
            const gptr<float> Ag = G(w.Aneg);
#pragma unroll
            for (int n = 0; n < FNS; n += 4) {
                const float4 p = ldg_f4(Ag + ((int64_t)(n / 4) * FDI + c) * 4);
                av[n] = p.x; av[n + 1] = p.y; av[n + 2] = p.z; av[n + 3] = p.w;
            }
#pragma unroll
            for (int r = 0; r < FR; r += 4) {
                const float4 q = ldg_f4(G(w.dt_w) + (int64_t)c * FR + r);
                wr[r] = q.x; wr[r + 1] = q.y; wr[r + 2] = q.z; wr[r + 3] = q.w;
            }
        }
        const float bdt = G(w.dt_b)[c], Dc = G(w.D)[c];
        // SSM state of this workgroup's valid lanes [b0, b0 + nb): rows past the last lane read 0 and are not
        // written (buffer range check).  No load or store is under a branch: the compiler's wait counts treat
        // a memory operation under a branch as possibly not issued, and every row would then wait for all
        // loads in flight.
        const __amdgpu_buffer_rsrc_t sr =
            buf_rsrc(a.ssm + ((int64_t)l * a.max_lanes + b0) * FDI * FNS, (uint32_t)nb * FDI * FNS * 4);
        auto h_off = [&](int r, int n, int cq) { return (uint32_t)((r * FNS / 4 + n / 4) * FDI + cq) * 16; };
        f32x4 h_first[FNS / 4];
        auto load_first = [&]() {
#pragma unroll
            for (int n = 0; n < FNS; n += 4) h_first[n / 4] = buf_ld4(sr, h_off(0, n, c));
        };
        if constexpr (HOIST_FIRST) load_first();
        // ---- x_proj fold: dbc = P_0 + P_1 + ... + P_7, in place of P_0 (element i is read and written by one
        //      thread only)
        for (int i = tid; i < ROWS * FW; i += NTHR) {
            float v = sPart[i];
#pragma unroll
            for (int q = 1; q < FDI / XPROJ_KB; ++q) v = v + sPart[q * (ROWS * FW) + i];
            sDbc[i] = v;
        }
        __syncthreads();
        // ---- dt_proj + softplus + selective scan + D + gate (thread = channel) -> y split operand
        {
            if constexpr (!HOIST_FIRST) load_first();
            // One lane's state at a time (lane 0's loaded before x_proj), stored at the end of its row.  The two waves
            // of a SIMD take turns waiting on memory.  In the split forms each row's state is loaded at the top of
            // the row (the barrier keeps the loads ahead of the row's LDS reads); keeping 1-3 more lanes in flight
            // per thread measured 2-7% slower there (more registers in a kernel at its register limit).
            // AHEAD (fp32 form, which has the registers): the next lane's state is loaded at the top of this row,
            // before this row's stores, so waiting for it (one in-order counter for loads and stores) does not wait
            // for those stores (0.3% per step; the same in the split forms)
            constexpr bool AHEAD = NT == 1;
            f32x4 hn[FNS / 4];
#pragma unroll
            for (int n = 0; n < FNS; n += 4) hn[n / 4] = h_first[n / 4];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                int cq = c;  // opaque per lane: offsets formed here, not held across the loop (see the conv)
                __asm__ volatile("" : "+v"(cq));
                float h[FNS];
#pragma unroll
                for (int n = 0; n < FNS; n += 4) {
                    const f32x4 q = AHEAD ? hn[n / 4] : (r == 0 ? h_first[n / 4] : buf_ld4(sr, h_off(r, n, cq)));
                    h[n] = q.x; h[n + 1] = q.y; h[n + 2] = q.z; h[n + 3] = q.w;
                }
                if constexpr (AHEAD) {
                    if (r + 1 < ROWS) {
#pragma unroll
                        for (int n = 0; n < FNS; n += 4) hn[n / 4] = buf_ld4(sr, h_off(r + 1, n, cq));
                    }
                }
                // the row's [dr | B | C] (uniform across the workgroup) into registers, all 12 reads issued together:
                // read where they are used, each waited for its own LDS round trip
                float dbc[FW];
                // the rows' LDS base in a register (opaque zero), so the 12 reads take immediate offsets instead of a
                // constant address materialised for each
                int zb = 0;
                __asm__ volatile("" : "+v"(zb));
                const float* rowp = sDbc + zb + r * FW;
#pragma unroll
                for (int i = 0; i < FW; i += 4) {
                    const float4 v = *reinterpret_cast<const float4*>(rowp + i);
                    dbc[i] = v.x; dbc[i + 1] = v.y; dbc[i + 2] = v.z; dbc[i + 3] = v.w;
                }
                __builtin_amdgcn_sched_barrier(0);
                const float x = sX[r * LXZ + cq], z = sX[r * LXZ + FDI + cq];
                const float y = scan_position<FNS, FR>(dbc, wr, bdt, av, Dc, x, z, h);
                store_op<NT, LA>(sAh, r, cq, y);
#pragma unroll
                for (int n = 0; n < FNS; n += 4)
                    buf_st4(sr, h_off(r, n, cq), f32x4{h[n], h[n + 1], h[n + 2], h[n + 3]});
            }
        }
        __syncthreads();
        // ---- out_proj (+bias) -> mixer output fp32 (stride LRES, in the xz region)
        {
            floatx4 acc[FPW_S];
            float bias_j[FPW_S];
#pragma unroll
            for (int j = 0; j < FPW_S; ++j) bias_j[j] = G(w.out_b)[16 * frag_of<NWAVE>(0, wave, j, FD / 16, rot16) + n_of];
            mgemm<NT, NWAVE, FPW_S, FDI, D_S, false>(sAh, sAl, LA, w.out_p, 0, FD / 16, wave, lane, rot16, acc);
#pragma unroll
            for (int j = 0; j < FPW_S; ++j) {
                const int n = 16 * frag_of<NWAVE>(0, wave, j, FD / 16, rot16) + n_of;
                const float bias = bias_j[j];
#pragma unroll
                for (int r = 0; r < 4; ++r) sX[(m_of + r) * LRES + n] = epi_value<EPI_BIAS>(acc[j][r], bias);
            }
        }
        lnw = ldg_f4(G(w.ln2_w) + 4 * lane);
        lnb = ldg_f4(G(w.ln2_b) + 4 * lane);
        __syncthreads();
        // ---- LN2 -> split operand
        ln_rows<NT, RPW>(sX, lnw, lnb, sAh, sAl, wave, lane);
        __syncthreads();
        // ---- FF1 (+bias, GELU) -> hidden split (xz region)
#pragma unroll 1
        for (int f0 = 0; f0 < 4 * FD / 16; f0 += FPW_B * NWAVE) {
            floatx4 acc[FPW_B];
            float bias_j[FPW_B];
#pragma unroll
            for (int j = 0; j < FPW_B; ++j) bias_j[j] = G(w.ff1_b)[16 * frag_of<NWAVE>(f0, wave, j, 4 * FD / 16, rot64) + n_of];
            mgemm<NT, NWAVE, FPW_B, FD, D_B, false, 2>(sAh, sAl, LA, w.ff1_p, f0, 4 * FD / 16, wave, lane, rot64, acc);
#pragma unroll
            for (int j = 0; j < FPW_B; ++j) {
                const int n = 16 * frag_of<NWAVE>(f0, wave, j, 4 * FD / 16, rot64) + n_of;
                const float bias = bias_j[j];
#pragma unroll
                for (int r = 0; r < 4; ++r) store_op<NT, LH>(sHh, m_of + r, n, epi_value<EPI_GELU>(acc[j][r], bias));
            }
        }
        __syncthreads();
        // ---- FF2 (+bias) + block residual -> residual stream
        {
            floatx4 acc[FPW_S];
            float bias_j[FPW_S];
#pragma unroll
            for (int j = 0; j < FPW_S; ++j) bias_j[j] = G(w.ff2_b)[16 * frag_of<NWAVE>(0, wave, j, FD / 16, rot16) + n_of];
            mgemm<NT, NWAVE, FPW_S, 4 * FD, D_S, false>(sHh, sHl, LH, w.ff2_p, 0, FD / 16, wave, lane, rot16, acc);
#pragma unroll
            for (int j = 0; j < FPW_S; ++j) {
                const int n = 16 * frag_of<NWAVE>(0, wave, j, FD / 16, rot16) + n_of;
                const float bias = bias_j[j];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int idx = (m_of + r) * LRES + n;
                    sRes[idx] = sRes[idx] + epi_value<EPI_RESID>(acc[j][r], bias);
                }
            }
        }
        {
            CFusedLayer& wn = layer_at(a.layers, l + 1 < a.L ? l + 1 : l);  // the last layer reloads its own (unused)
            lnw = ldg_f4(G(wn.ln1_w) + 4 * lane);
            lnb = ldg_f4(G(wn.ln1_b) + 4 * lane);
        }
        __syncthreads();
    }

    // ---- head: Linear -> ReLU -> Linear (model.py:95, 101); lane values from an opaque copy, as in the layer loop
    int tid_h = (int)threadIdx.x;
    if constexpr (NT == 1) __asm__ volatile("" : "+v"(tid_h));
    const int tid = tid_h, lane = tid_h & 63;
    const int m_of = 4 * (lane >> 4), n_of = lane & 15;
    for (int i = tid; i < ROWS * FD; i += NTHR) {
        const int r = i / FD, c = i % FD;
        store_op<NT, LA>(sAh, r, c, sRes[r * LRES + c]);
    }
    __syncthreads();
    uint16_t* sGh = sHh;
    uint16_t* sGl = sHh + ROWS * LH1;
    {
        floatx4 acc[FPW_S];
        mgemm<NT, NWAVE, FPW_S, FD, D_S, false>(sAh, sAl, LA, a.h1_p, 0, FD / 16, wave, lane, rot16, acc);
#pragma unroll
        for (int j = 0; j < FPW_S; ++j) {
            const int n = 16 * frag_of<NWAVE>(0, wave, j, FD / 16, rot16) + n_of;
            const float bias = G(a.h1_b)[n];
#pragma unroll
            for (int r = 0; r < 4; ++r) store_op<NT, LH1>(sGh, m_of + r, n, epi_value<EPI_RELU>(acc[j][r], bias));
        }
    }
    __syncthreads();
    {
        floatx4 acc[FPW_S];
        // a full 256-symbol vocabulary covers every fragment (no per-fragment condition); smaller ones check
        if (V == FPW_S * NWAVE * 16)
            mgemm<NT, NWAVE, FPW_S, FD, D_S, false>(sGh, sGl, LH1, a.h2_p, 0, V / 16, wave, lane, 0, acc);
        else
            mgemm<NT, NWAVE, FPW_S, FD, D_S>(sGh, sGl, LH1, a.h2_p, 0, V / 16, wave, lane, 0, acc);
#pragma unroll
        for (int j = 0; j < FPW_S; ++j) {
            const int f = wave + NWAVE * j;
            if (f < V / 16) {
                const int n = 16 * f + n_of;
                const float bias = G(a.h2_b)[n];
#pragma unroll
                for (int r = 0; r < 4; ++r) sLog[(m_of + r) * LRES + n] = epi_value<EPI_BIAS>(acc[j][r], bias);
            }
        }
    }
    __syncthreads();
    if (a.logits) {
        for (int i = tid; i < ROWS * V; i += NTHR) {
            const int r = i / V, n = i % V;
            if (r < nb) a.logits[(b0 + r) * V + n] = sLog[r * LRES + n];
        }
    }
    if (a.decode) {
#pragma unroll
        for (int q = 0; q < RPW; ++q) {
            const int r = RPW * wave + q;
            if (r >= nb) continue;
            const int64_t b = b0 + r;
            if (t >= a.lens[b]) continue;
            DecState st = a.dec[b];
            const LaneWords w = lane_words(a.payload, a.payload_words, a.off, a.nwords, b);
            const int s = decode_row(sLog + r * LRES, V, lane, st, w.p, w.n);
            if (lane == 0) {
                a.dec[b] = st;
                sTok[r] = s;
                a.out[b * a.out_stride + t] = (uint8_t)s;
            }
        }
    }
    __syncthreads();  // next step reads sTok, and sLog's region is reused
    p0m3 = p0m3 == 2 ? 0 : p0m3 + 1;
    }
    if (a.decode && tid < nb) a.tokens_out[b0 + tid] = sTok[tid];
}

}  // namespace

bool fused_step_supported(int d_model, int d_state, int dt_rank, int d_conv, int vocab) {
    return d_model == FD && d_state == FNS && dt_rank == FR && d_conv == 4 && vocab % 16 == 0 && vocab <= 256;
}

hipError_t launch_fused_step(const FusedArgs& a, int nt, hipStream_t s) {
    const dim3 grid((unsigned)((a.B + ROWS - 1) / ROWS));
    if (nt == 3) hipLaunchKernelGGL((k_fused_step<3, 512>), grid, dim3(512), 0, s, a);
    else if (nt == 2) hipLaunchKernelGGL((k_fused_step<2, 512>), grid, dim3(512), 0, s, a);
    else hipLaunchKernelGGL((k_fused_step<1, 512>), grid, dim3(512), 0, s, a);
    return hipGetLastError();
}

}  // namespace boa
