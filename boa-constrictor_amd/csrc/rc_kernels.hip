// Range-coder kernels of libboa_hip.so: the coder on precomputed tables (range coder alone), the per-step
// batch coder with the reference's Q2 quantiser (drop-in for gpu.queue.RangeCoderBatch; its word export
// goes through boa_compact, compact.hip), and the fused quantiser's table export used by the parity tests.
//
// One chunk lane per stream throughout.  Wave-parallel work (table search, Q2 prefix sums, quantiser scans) is
// done by one 64-wide wavefront per lane, or, in the throughput decoders on full tables, by 8 or 16 lanes per
// stream (8 or 4 streams per wavefront); the coder state itself is uniform across a stream's lanes.
#include "boa_common.h"

#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>
#include <string>
#include <type_traits>
#include <vector>

#include "../../include/boa_hip.h"

using namespace boa;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ================================================================================================
// Coder on precomputed tables.  Table row = cdf[0..K-1] of one step (cdf[K] = 2^P implied).

template <int P, typename TC>
__global__ void __launch_bounds__(256) k_rc_encode_tables(const TC* __restrict__ cdf, int K,
                                                         const uint8_t* __restrict__ syms, int streams,
                                                         int len, uint32_t* __restrict__ words,
                                                         int64_t pitch, int32_t* __restrict__ nwords) {
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= streams) return;
    EncState st;
    enc_init(st);
    const WordSink sink{words + (int64_t)n * pitch, pitch, true};
    const TC* c = cdf + (int64_t)n * len * K;
    const uint8_t* s = syms + (int64_t)n * len;
    for (int t = 0; t < len; ++t) {
        const int sym = s[t];
        if (sym >= K) continue;  // gpu_range_coder.py:97: symbols outside [0, K) are skipped
        const uint32_t lo = (uint32_t)c[(int64_t)t * K + sym];
        const uint32_t hi = (sym + 1 < K) ? (uint32_t)c[(int64_t)t * K + sym + 1] : (1u << P);
        enc_push(st, P, lo, hi - lo, sink);
    }
    enc_finish(st, sink);
    nwords[n] = st.nwords;  // > pitch signals overflow (nothing past the pitch was written)
}

template <int P, typename TC>
__global__ void __launch_bounds__(64) k_rc_decode_tables(const TC* __restrict__ cdf, int K,
                                                        const uint32_t* __restrict__ words, int64_t pitch,
                                                        const int32_t* __restrict__ nwords, int streams,
                                                        int len, uint8_t* __restrict__ syms) {
    const int n = blockIdx.x;
    const int lane = threadIdx.x;
    if (n >= streams) return;
    const uint32_t* in = words + (int64_t)n * pitch;
    int32_t nw = nwords[n];
    if (nw > pitch) nw = (int32_t)pitch;
    DecState st;
    dec_init(st, in, nw);
    const TC* c = cdf + (int64_t)n * len * K;
    uint32_t cur[4], nxt[4];
    if (len > 0) load_row4<P>(c, K, lane, cur);
    for (int t = 0; t < len; ++t) {
        if (t + 1 < len) load_row4<P>(c + (int64_t)(t + 1) * K, K, lane, nxt);
        const uint32_t q = dec_target(st, P);
        uint32_t lo, hi;
        const int s = wave_find_symbol<P>(cur, K, q, lane, lo, hi);
        if (lane == 0) syms[(int64_t)n * len + t] = (uint8_t)s;
        dec_advance(st, P, lo, hi - lo, in, nw);
#pragma unroll
        for (int j = 0; j < 4; ++j) cur[j] = nxt[j];
    }
}

// Keeps memory operations in program order across this point (a compiler barrier, no instruction): a register
// ring's loads stay issued oldest row first, so the wait counts the compiler places before each row's use (the
// loads outstanding after it, the same on loop entry as on every later pass) leave the newer rows in flight.
__device__ __forceinline__ void pin_order() { asm volatile("" ::: "memory"); }
// Word 3 of a raw buffer descriptor on gfx950 (32-bit data format): accesses past num_records bytes read 0 and
// drop their stores.
constexpr int BUF_DESC_WORD3 = 0x00020000;
typedef uint32_t u32x2v __attribute__((vector_size(8)));
constexpr int ROW_CPOL = 2;  // cache policy of the table row loads: NT (non-temporal)

// DPP moves inside rows of 16 lanes: fixed lane permutations applied as an operand of a VALU instruction, with
// no LDS round trip (the ds_bpermute behind __shfl is one).  A lane whose source is outside its row reads 0.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}
constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1, 0, 3, 2]: lane i <- lane i ^ 1
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2, 3, 0, 1]: lane i <- lane i ^ 2
constexpr int DPP_HALF_MIRROR = 0x141; // row_half_mirror: lane i <- lane 7 - i within each 8 lanes
constexpr int DPP_SHR1 = 0x111;        // row_shr:1: lane i <- lane i - 1 within each 16 lanes
constexpr int DPP_MIRROR = 0x140;      // row_mirror: lane i <- lane 15 - i within each 16 lanes

// The same coder for full tables (K = 256) in any table format, lengths divisible by D: four streams per
// wavefront, 16 lanes per stream, lane j holding entries 16 j .. 16 j + 15 of each row (a row of one stream is
// one contiguous 512 B (2-byte entries) or 1 KiB (4-byte entries) read by its 16 lanes).  The scaffolding is
// k_rc_decode_tables8's (below): rows through a non-temporal register ring D - 1 steps ahead, code words from a
// three-block register window moved once per pass, symbols stored once per pass, no memory access under a
// branch.  The coder arithmetic is the reference's (rc_core.h: dec_target, and dec_advance's update with its
// word from the window; gpu_range_coder.py:182-210); the symbol search keeps its semantics (the smallest i in
// [1, K] with cdf[i] > q, minus one): each lane finds its first such entry in one pass from the top, carrying
// cdf[i] and cdf[i - 1]; the stream's smallest index, then that entry's two values, are reduced over its 16
// lanes with DPP moves (no entry > q gives index K, with cdf[K - 1] from the last lane and hi = 2^P).
template <int P, typename TC, int D = 4>
__global__ void __launch_bounds__(256) k_rc_decode_tables4(const TC* __restrict__ cdf,
                                                         const uint32_t* __restrict__ words, int64_t pitch,
                                                         const int32_t* __restrict__ nwords, int streams, int len,
                                                         uint8_t* __restrict__ syms, uint32_t words_bytes) {
    constexpr int K = 256, S = 16, E = K / S, G = 64 / S;
    constexpr int NV = E * (int)sizeof(TC) / 16;  // 16-byte loads per lane per row
    constexpr uint32_t ROWB = K * sizeof(TC);      // bytes per row
    static_assert(D <= S, "at most S words are read per pass of D steps");
    const int lane = threadIdx.x & 63;
    const int j = lane & (S - 1), gbase = lane & ~(S - 1);
    const int64_t n = ((int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6)) * G + lane / S;
    const bool live = n < streams;
    const int64_t nn = live ? n : 0;  // streams past the last shadow stream 0 with no words and write nothing
    int32_t nw = live ? nwords[nn] : 0;
    if (nw > pitch) nw = (int32_t)pitch;
    DecState st;
    dec_init(st, words + nn * pitch, nw);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(words), (short)0,
                                                                        (int)(words_bytes), BUF_DESC_WORD3);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(syms, (short)0, (int)((uint32_t)streams * (uint32_t)len), BUF_DESC_WORD3);
    const uint32_t wbase = (uint32_t)(nn * pitch) * 4u;
    auto word = [&](int i) {
        return __builtin_amdgcn_raw_buffer_load_b32(rw, i < nw ? wbase + (uint32_t)i * 4u : 0xFFFFFFF0u, 0, 0);
    };
    const uint32_t sbase = (uint32_t)((live ? nn : (int64_t)streams) * len);
    int32_t base = 0;
    uint32_t w0 = word(j), w1 = word(S + j), w2 = word(2 * S + j);
    const int64_t wfirst =
        ((int64_t)blockIdx.x * (blockDim.x / 64) + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6))) * G;
    const int nlive = (int)(streams - wfirst < 0 ? 0 : (streams - wfirst > G ? G : streams - wfirst));
    const __amdgpu_buffer_rsrc_t rt = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<TC*>(cdf + (nlive > 0 ? wfirst : 0) * (int64_t)len * K), (short)0,
        (int)((uint32_t)nlive * (uint32_t)len * ROWB), BUF_DESC_WORD3);
    const uint32_t tbase = (uint32_t)(lane / S) * (uint32_t)len * ROWB + (uint32_t)(E * sizeof(TC)) * (uint32_t)j;
    u32x4 rows[D][NV];
    auto load_row = [&](int t, u32x4 (&r)[NV]) {
        const uint32_t o = tbase + (uint32_t)(t < len ? t : len - 1) * ROWB;
#pragma unroll
        for (int v = 0; v < NV; ++v)
            r[v] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rt, o + 16u * v, 0, ROW_CPOL));
    };
#pragma unroll
    for (int u = 0; u < D - 1; ++u) {
        load_row(u, rows[u]);
        pin_order();
    }
#pragma unroll 1
    for (int t0 = 0; t0 < len; t0 += D) {
        const bool rot = st.read_idx - base >= S;
        w0 = rot ? w1 : w0;
        w1 = rot ? w2 : w1;
        base += rot ? S : 0;
        w2 = word(base + 2 * S + j);
        uint32_t packed = 0;
#pragma unroll
        for (int u = 0; u < D; ++u) {
            load_row(t0 + u + D - 1, rows[(u + D - 1) % D]);
            pin_order();
            const int o = st.read_idx - base;  // 0 <= o < 2S
            const uint32_t wa =
                (uint32_t)__builtin_amdgcn_ds_bpermute((gbase + (o & (S - 1))) * 4, (int)(o < S ? w0 : w1));
            uint32_t e[E];
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const uint32_t d[4] = {rows[u][v].x, rows[u][v].y, rows[u][v].z, rows[u][v].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if constexpr (sizeof(TC) == 2) {
                        e[8 * v + 2 * k] = d[k] & 0xFFFFu;
                        e[8 * v + 2 * k + 1] = d[k] >> 16;
                    } else {
                        e[4 * v + k] = d[k];
                    }
                }
            }
            const uint32_t q = P <= 16 ? dec_target16(st, P) : dec_target(st, P);
            const uint32_t prev_last = dpp<DPP_SHR1>(e[E - 1]);  // cdf[E j - 1] (unused for j = 0)
            int first = E;
            uint32_t hv = j == S - 1 ? (1u << P) : 0u, lv = j == S - 1 ? e[E - 1] : 0u;  // index K: last lane
#pragma unroll
            for (int i = E - 1; i >= 0; --i) {
                const bool pred = e[i] > q && (i > 0 || j > 0);
                first = pred ? i : first;
                hv = pred ? e[i] : hv;
                lv = pred ? (i > 0 ? e[i - 1] : prev_last) : lv;
            }
            const int cand = first < E ? E * j + first : (j == S - 1 ? K : K + 1);
            int kl = cand;
            kl = min(kl, (int)dpp<DPP_XOR1>((uint32_t)kl));
            kl = min(kl, (int)dpp<DPP_XOR2>((uint32_t)kl));
            kl = min(kl, (int)dpp<DPP_HALF_MIRROR>((uint32_t)kl));
            kl = min(kl, (int)dpp<DPP_MIRROR>((uint32_t)kl));
            const bool own = cand == kl;
            uint32_t lo = own ? lv : 0u, hi = own ? hv : 0u;
            lo |= dpp<DPP_XOR1>(lo);
            hi |= dpp<DPP_XOR1>(hi);
            lo |= dpp<DPP_XOR2>(lo);
            hi |= dpp<DPP_XOR2>(hi);
            lo |= dpp<DPP_HALF_MIRROR>(lo);
            hi |= dpp<DPP_HALF_MIRROR>(hi);
            lo |= dpp<DPP_MIRROR>(lo);
            hi |= dpp<DPP_MIRROR>(hi);
            packed |= (uint32_t)(uint8_t)(kl - 1) << (8 * u);
            // dec_advance (rc_core.h), one renormalisation at most: the range is >= 2^32 before every step, so
            // range' = (range >> P) * prob >= 2^(32 - P) and one 32-bit shift restores range >= 2^32
            uint32_t prob = hi - lo;
            if (prob == 0u) prob = 1u;
            const uint64_t scale = st.range >> P;
            st.lower = st.lower + scale * (uint64_t)lo;
            st.range = scale * (uint64_t)prob;
            const bool sh = st.range < (1ull << 32);
            st.lower = sh ? st.lower << 32 : st.lower;
            st.range = sh ? st.range << 32 : st.range;
            st.point = sh ? (st.point << 32) | (uint64_t)wa : st.point;
            st.read_idx += (sh && st.read_idx < nw) ? 1 : 0;
        }
        __builtin_amdgcn_raw_buffer_store_b32(packed, rs, sbase + (uint32_t)t0, 0, 0);
    }
}


// The table decoder for 2-byte tables at P = 16 (configs[1]'s coder), K = 256, lengths divisible by D: eight
// lanes per stream, so eight streams per wavefront and half the instructions per decoded symbol of the
// four-streams form above.  Lane j of a stream holds entries 64 v + 8 j .. + 7 (v = 0..3) of each row, so each
// of its four 16-byte loads is, over the stream's eight lanes, one contiguous 128-byte line of the row; rows
// are prefetched D - 1 steps ahead through a register ring.  Per step:
//  - each entry i >= 1 is tested as a pair word (cdf[i] << 16) | cdf[i - 1] against (q << 16) | 0xFFFF, which
//    it exceeds exactly when cdf[i] > q (cdf[i - 1] <= 0xFFFF); a lane keeps its first such entry's index and
//    pair word (the pair word of entry 2m is one funnel shift of two table dwords, that of entry 2m + 1 a dword);
//  - the stream's smallest index over its eight lanes, then that entry's pair word (from the one lane that
//    holds it, the others contributing 0), are reduced with DPP moves; no entry > q gives index K, with
//    cdf[K - 1] from the stream's last lane and hi = 2^P;
//  - the symbol is that index minus one (the reference's linear search, gpu_range_coder.py:195-199), and the
//    coder update is dec_advance's (rc_core.h), its renormalisation word read from the register window before
//    the search (the window's first half always holds it: the read position stays within S words of its base).
// The D symbols of a pass are stored as one D-byte word.
template <int D>
__global__ void __launch_bounds__(256) k_rc_decode_tables8(const uint16_t* __restrict__ cdf,
                                                         const uint32_t* __restrict__ words, int64_t pitch,
                                                         const int32_t* __restrict__ nwords, int streams, int len,
                                                         uint8_t* __restrict__ syms, uint32_t words_bytes) {
    constexpr int P = 16, K = 256, S = 8, NV = 4, E = 32;  // lanes per stream, 16-byte loads and entries per lane
    static_assert(D == 4 || D == 8, "symbols of a pass are stored as one 4- or 8-byte word");
    using SymWord = typename std::conditional<D == 8, uint64_t, uint32_t>::type;
    const int lane = threadIdx.x & 63;
    const int j = lane & (S - 1), gbase = lane & ~(S - 1);
    const int64_t n = ((int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6)) * (64 / S) + lane / S;
    const bool live = n < streams;
    const int64_t nn = live ? n : 0;  // streams past the last shadow stream 0 with no words and write nothing
    const uint32_t* in = words + nn * pitch;
    int32_t nw = live ? nwords[nn] : 0;
    if (nw > pitch) nw = (int32_t)pitch;
    DecState st;
    dec_init(st, in, nw);
    // Code words and symbols through buffer descriptors over the whole word and symbol arrays (the launch
    // checks that both fit 32-bit byte offsets); a word past the stream's nw (read as 0, as dec_advance does)
    // and a shadow stream's symbols take an offset past the end, which reads 0 and drops the store.  So no
    // access in the loop is under a branch, and the compiler's wait before each row's use counts exactly the
    // loads issued after it: the rows behind it stay in flight.
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(words), (short)0,
                                                                        (int)(words_bytes), BUF_DESC_WORD3);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(syms, (short)0, (int)((uint32_t)streams * (uint32_t)len), BUF_DESC_WORD3);
    const uint32_t wbase = (uint32_t)(nn * pitch) * 4u;
    auto word = [&](int i) {
        return __builtin_amdgcn_raw_buffer_load_b32(rw, i < nw ? wbase + (uint32_t)i * 4u : 0xFFFFFFF0u, 0, 0);
    };
    // a shadow stream's stores start at the end of the array (the launch keeps (streams + 1) * len below 2^32)
    const uint32_t sbase = (uint32_t)((live ? nn : (int64_t)streams) * len);
    // window of three blocks of S words: lane j holds words base + j, base + S + j, base + 2S + j
    int32_t base = 0;
    uint32_t w0 = word(j), w1 = word(S + j), w2 = word(2 * S + j);
    // Table rows through a descriptor over the tables of this wavefront's eight streams (the launch keeps 8 len
    // rows of 512 B below 2^32 bytes): the rows of a stream past the last are past its end and read 0.  The loads
    // are non-temporal: every row is read once, and streaming it past the caches measured 17% faster.
    const int64_t wfirst =
        ((int64_t)blockIdx.x * (blockDim.x / 64) + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6))) * (64 / S);
    const int nlive = (int)(streams - wfirst < 0 ? 0 : (streams - wfirst > 64 / S ? 64 / S : streams - wfirst));
    const __amdgpu_buffer_rsrc_t rt = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(cdf + (nlive > 0 ? wfirst : 0) * (int64_t)len * K), (short)0,
        (int)((uint32_t)nlive * (uint32_t)len * (uint32_t)(K * 2)), BUF_DESC_WORD3);
    const uint32_t tbase = (uint32_t)(lane / S) * (uint32_t)len * (uint32_t)(K * 2) + 16u * (uint32_t)j;
    u32x4 rows[D][NV];
    auto load_row = [&](int t, u32x4 (&r)[NV]) {
        const uint32_t o = tbase + (uint32_t)(t < len ? t : len - 1) * (uint32_t)(K * 2);
#pragma unroll
        for (int v = 0; v < NV; ++v)
            r[v] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rt, o + 128u * v, 0, ROW_CPOL));
    };
#pragma unroll
    for (int u = 0; u < D - 1; ++u) {
        load_row(u, rows[u]);
        pin_order();
    }
#pragma unroll 1
    for (int t0 = 0; t0 < len; t0 += D) {
        // at most D <= S words are read per pass: once the read position has left the window's first block, the
        // window moves by one block (its third, fetched a pass ago), and the block after it is fetched
        const bool rot = st.read_idx - base >= S;
        w0 = rot ? w1 : w0;
        w1 = rot ? w2 : w1;
        base += rot ? S : 0;
        w2 = word(base + 2 * S + j);
        SymWord packed = 0;
#pragma unroll
        for (int u = 0; u < D; ++u) {
            load_row(t0 + u + D - 1, rows[(u + D - 1) % D]);
            pin_order();
            const int o = st.read_idx - base;  // 0 <= o < 2S
            const uint32_t wa =
                (uint32_t)__builtin_amdgcn_ds_bpermute((gbase + (o & (S - 1))) * 4, (int)(o < S ? w0 : w1));
            const uint32_t q = dec_target16(st, P);
            const uint32_t qk = (q << 16) | 0xFFFFu;
            uint32_t sel = j == S - 1 ? rows[u][NV - 1].w >> 16 : 0u;  // cdf[K - 1], for index K
            int first = E;                                             // local index 8 v + k; E: none
#pragma unroll
            for (int v = NV - 1; v >= 0; --v) {
                const uint32_t dv[4] = {rows[u][v].x, rows[u][v].y, rows[u][v].z, rows[u][v].w};
                // dword holding entry 64 v + 8 j - 1 in its high half: lane j - 1's last of this chunk, for lane 0
                // lane 7's last of the chunk before (global entry 0 has none and is not tested)
                const uint32_t prev_same = dpp<DPP_SHR1>(dv[3]);
                const uint32_t prev_wrap = v > 0 ? dpp<DPP_HALF_MIRROR>(rows[u][v - 1].w) : 0u;
                const uint32_t pv = j > 0 ? prev_same : prev_wrap;
#pragma unroll
                for (int k = 7; k >= 0; --k) {
                    const int m = k >> 1;
                    const uint32_t pw = (k & 1) ? dv[m] : __builtin_amdgcn_alignbit(dv[m], m > 0 ? dv[m - 1] : pv, 16);
                    const bool pred = pw > qk && (v > 0 || k > 0 || j > 0);
                    sel = pred ? pw : sel;
                    first = pred ? 8 * v + k : first;
                }
            }
            const int cand = first < E ? 64 * (first >> 3) + 8 * j + (first & 7) : (j == S - 1 ? K : K + 1);
            int kl = cand;
            kl = min(kl, (int)dpp<DPP_XOR1>((uint32_t)kl));
            kl = min(kl, (int)dpp<DPP_XOR2>((uint32_t)kl));
            kl = min(kl, (int)dpp<DPP_HALF_MIRROR>((uint32_t)kl));
            uint32_t vv = cand == kl ? sel : 0u;
            vv |= dpp<DPP_XOR1>(vv);
            vv |= dpp<DPP_XOR2>(vv);
            vv |= dpp<DPP_HALF_MIRROR>(vv);
            const uint32_t lo = vv & 0xFFFFu;
            const uint32_t hi = kl < K ? vv >> 16 : (1u << P);
            packed |= (SymWord)(uint8_t)(kl - 1) << (8 * u);
            // dec_advance (rc_core.h), one renormalisation at most (the range is >= 2^32 before every step)
            uint32_t prob = hi - lo;
            if (prob == 0u) prob = 1u;
            const uint64_t scale = st.range >> P;
            st.lower = st.lower + scale * (uint64_t)lo;
            st.range = scale * (uint64_t)prob;
            const bool sh = st.range < (1ull << 32);
            st.lower = sh ? st.lower << 32 : st.lower;
            st.range = sh ? st.range << 32 : st.range;
            st.point = sh ? (st.point << 32) | (uint64_t)wa : st.point;
            st.read_idx += (sh && st.read_idx < nw) ? 1 : 0;
        }
        // the stream's eight lanes store the same word (one write)
        if constexpr (D == 8)
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2v, packed), rs, sbase + (uint32_t)t0, 0, 0);
        else
            __builtin_amdgcn_raw_buffer_store_b32(packed, rs, sbase + (uint32_t)t0, 0, 0);
    }
}

constexpr int ENC_LANES_PER_STREAM = 8;

// Encoder on full tables (K = 256), streams of a length divisible by 16: R lanes per stream, all computing the
// stream's coder state and the first of them writing its words, so that there are R times as many wavefronts
// as with one lane per stream (a wavefront's symbols are a sequential chain of dependent steps; more wavefronts
// per SIMD hide more of its latency; 8 lanes measured 12% faster than 1).  The table entries of 16 symbols
// (independent of the coder state) are loaded one block ahead, non-temporal (6% faster: each is read once), the
// symbols two blocks ahead, so enc_push (rc_core.h) runs without waiting on memory.
template <int P, typename TC, int R>
__global__ void __launch_bounds__(64) k_rc_encode_tables16(const TC* __restrict__ cdf,
                                                         const uint8_t* __restrict__ syms, int streams, int len,
                                                         uint32_t* __restrict__ words, int64_t pitch,
                                                         int32_t* __restrict__ nwords) {
    constexpr int K = 256, B = 16;
    const int64_t n = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / R;
    const bool live = n < streams;
    const bool writer = live && threadIdx.x % R == 0;
    const int64_t nn = live ? n : 0;
    EncState st;
    enc_init(st);
    const WordSink sink{words + nn * pitch, pitch, writer};
    const TC* c = cdf + nn * (int64_t)len * K;
    const uint8_t* sp = syms + nn * (int64_t)len;
    const int nb = len / B;
    auto load_syms = [&](int b) { return *reinterpret_cast<const uint4*>(sp + (int64_t)(b < nb ? b : nb - 1) * B); };
    auto issue = [&](int b, uint4 sv, uint32_t (&lo)[B], uint32_t (&hi)[B]) {
        const int bb = b < nb ? b : nb - 1;
        const uint32_t w[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int s = (w[u / 4] >> (8 * (u % 4))) & 0xFF;
            const TC* r = c + ((int64_t)bb * B + u) * K;
            lo[u] = (uint32_t)__builtin_nontemporal_load(r + s);
            hi[u] = (uint32_t)__builtin_nontemporal_load(r + (s + 1 < K ? s + 1 : s));
            if (s + 1 >= K) hi[u] = 1u << P;
        }
    };
    auto code = [&](const uint32_t (&lo)[B], const uint32_t (&hi)[B]) {
#pragma unroll
        for (int u = 0; u < B; ++u) enc_push(st, P, lo[u], hi[u] - lo[u], sink);
    };
    uint32_t loA[B], hiA[B], loB[B], hiB[B];
    uint4 sv1 = load_syms(1), sv2;
    issue(0, load_syms(0), loA, hiA);
#pragma unroll 1
    for (int b = 0; b < nb; b += 2) {
        sv2 = load_syms(b + 2);
        issue(b + 1, sv1, loB, hiB);
        code(loA, hiA);
        if (b + 1 >= nb) break;
        sv1 = load_syms(b + 3);
        issue(b + 2, sv2, loA, hiA);
        code(loB, hiB);
    }
    enc_finish(st, sink);
    if (writer) nwords[n] = st.nwords;
}

// ------------------------------------------------------------------------------------------------
// Synthetic tables: counter-based generator (SplitMix64 finaliser, Steele/Lea/Flood 2014) keyed by
// (seed, stream, step, index), Box-Muller normals, fused quantiser, inverse-CDF symbol draw.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

template <int P, typename TC>
__global__ void __launch_bounds__(256) k_rc_synth_tables(uint64_t seed, float sigma, int K, int streams,
                                                        int len, TC* __restrict__ cdf,
                                                        uint8_t* __restrict__ syms) {
    const int lane = threadIdx.x & 63;
    const int64_t rows = (int64_t)streams * len;
    const int64_t wave0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
    for (int64_t r = wave0; r < rows; r += nwaves) {
        const uint64_t key = mix64(seed ^ mix64((uint64_t)r));
        float l[4];
#pragma unroll
        for (int j = 0; j < 4; j += 2) {
            const uint64_t h = mix64(key + (uint64_t)(4 * lane + j));
            const float u1 = ((float)(uint32_t)(h >> 40) + 1.0f) * 0x1p-24f;      // (0, 1]
            const float u2 = (float)(uint32_t)(h & 0xFFFFFFu) * 0x1p-24f;         // [0, 1)
            const float rad = sqrtf(-2.0f * logf(u1));
            l[j] = sigma * rad * cosf(6.28318530718f * u2);
            l[j + 1] = sigma * rad * sinf(6.28318530718f * u2);
        }
        XQ q;
        xq_build(q, make_float4(l[0], l[1], l[2], l[3]), lane, K, P);
        uint32_t e[4];
        uint32_t c = q.base;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = 4 * lane + j;
            e[j] = (k < K) ? xq_cdf_at(q, c, k) : (1u << P);
            c += q.f[j];
        }
        TC* row = cdf + r * K;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = 4 * lane + j;
            if (k < K) row[k] = (TC)e[j];
        }
        const uint32_t u = (uint32_t)(mix64(key ^ 0x5851F42D4C957F2Dull) >> 20) & ((1u << P) - 1u);
        uint32_t lo, hi;
        const int s = wave_find_symbol<P>(e, K, u, lane, lo, hi);
        if (lane == 0) syms[r] = (uint8_t)s;
    }
}

// ================================================================================================
// Per-step batch coder, Q2 quantiser (gpu_range_coder.py:57-79) at PRECISION 24.

static constexpr int RCB_P = 24;
static constexpr int RCB_KMAX = 1024;  // the reference's per-thread table holds K+1 <= 1025 entries

__global__ void k_rcb_init(EncState* st, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) enc_init(st[i]);
}

// gpu_range_coder.py:88-141, one wavefront per lane: the probabilities are staged through LDS with
// coalesced loads, then lane 0 runs the sequential double accumulation of build_cdf_fast (the same
// additions in the same order, so the prefix values equal the reference's cumulative_float).
__global__ void __launch_bounds__(64) k_rcb_encode_step(const int32_t* __restrict__ syms,
                                                       const float* __restrict__ probs,
                                                       const uint8_t* __restrict__ mask, int n, int K,
                                                       EncState* __restrict__ states,
                                                       uint32_t* __restrict__ words, int64_t pitch) {
    __shared__ float sp[RCB_KMAX];
    const int b = blockIdx.x;
    const int lane = threadIdx.x;
    if (b >= n) return;
    if (mask && mask[b] == 0) return;
    const int s = syms[b];
    if (s < 0 || s >= K) return;
    const float* row = probs + (int64_t)b * K;
    for (int i = lane; i < K; i += 64) sp[i] = row[i];
    __syncthreads();
    if (lane != 0) return;
    const uint32_t TOTAL = 1u << RCB_P;
    const uint32_t free_weight = TOTAL - (uint32_t)K;
    double norm = 0.0, cum_s = 0.0, cum_s1 = 0.0;
    for (int i = 0; i < K; ++i) {
        if (i == s) cum_s = norm;
        if (i == s + 1) cum_s1 = norm;
        norm += (double)sp[i];
    }
    uint32_t lo, hi;
    if (!(norm > 0.0) || !__builtin_isfinite(norm)) {
        const uint32_t step = free_weight / (uint32_t)K + 1u;
        lo = (uint32_t)s * step;
        hi = (s + 1 < K) ? (uint32_t)(s + 1) * step : TOTAL;
    } else {
        const double scale = (double)free_weight / norm;
        lo = (uint32_t)(cum_s * scale) + (uint32_t)s;
        hi = (s + 1 < K) ? (uint32_t)(cum_s1 * scale) + (uint32_t)(s + 1) : TOTAL;
    }
    EncState st = states[b];
    const WordSink sink{words + (int64_t)b * pitch, pitch, true};
    enc_push(st, RCB_P, lo, hi - lo, sink);
    states[b] = st;
}

__global__ void k_rcb_finalize(EncState* states, uint32_t* words, int64_t pitch, int32_t* sizes, int n) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n) return;
    EncState st = states[b];
    const WordSink sink{words + (int64_t)b * pitch, pitch, true};
    enc_finish(st, sink);
    states[b] = st;
    sizes[b] = st.overflow ? -st.nwords : st.nwords;  // negative: the stream needed more than the pitch
}

__global__ void k_rcb_init_dec(DecState* states, const uint32_t* words, int64_t pitch,
                               const int32_t* sizes, int n) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n) return;
    DecState st;
    dec_init(st, words + (int64_t)b * pitch, sizes[b]);
    states[b] = st;
}

// gpu_range_coder.py:182-210.  Lane 0 writes the sequential Q2 prefix sums to LDS; the wave then
// evaluates every cdf entry in parallel and finds the reference's linear-search answer with ballots.
__global__ void __launch_bounds__(64) k_rcb_decode_step(const float* __restrict__ probs,
                                                       const uint8_t* __restrict__ mask, int n, int K,
                                                       DecState* __restrict__ states,
                                                       const uint32_t* __restrict__ words, int64_t pitch,
                                                       const int32_t* __restrict__ sizes,
                                                       int32_t* __restrict__ out_syms) {
    __shared__ float sp[RCB_KMAX];
    __shared__ double scum[RCB_KMAX + 1];
    __shared__ double s_scale;
    __shared__ int s_uniform;
    const int b = blockIdx.x;
    const int lane = threadIdx.x;
    if (b >= n) return;
    if (mask && mask[b] == 0) return;
    const float* row = probs + (int64_t)b * K;
    for (int i = lane; i < K; i += 64) sp[i] = row[i];
    __syncthreads();
    const uint32_t TOTAL = 1u << RCB_P;
    const uint32_t free_weight = TOTAL - (uint32_t)K;
    if (lane == 0) {
        double norm = 0.0;
        for (int i = 0; i < K; ++i) {
            scum[i] = norm;
            norm += (double)sp[i];
        }
        scum[K] = norm;
        const int uni = (!(norm > 0.0) || !__builtin_isfinite(norm)) ? 1 : 0;
        s_uniform = uni;
        s_scale = uni ? 0.0 : (double)free_weight / norm;
    }
    __syncthreads();
    const uint32_t* in = words + (int64_t)b * pitch;
    const int32_t nw = sizes[b];
    DecState st = states[b];
    const uint32_t q = dec_target(st, RCB_P);
    const bool uni = s_uniform != 0;
    const double scale = s_scale;
    const uint32_t ustep = free_weight / (uint32_t)K + 1u;
    auto cdf_at = [&](int i) -> uint32_t {
        if (i >= K) return TOTAL;
        if (uni) return (uint32_t)i * ustep;
        return (uint32_t)(scum[i] * scale) + (uint32_t)i;
    };
    // smallest i in [1, K] with cdf[i] > q
    int first = K;
    for (int base = 0; base < K; base += 64) {
        const int i = base + lane;
        const bool pred = (i >= 1) && (i < K) && (cdf_at(i) > q);
        const uint64_t m = __ballot(pred);
        if (m) { first = base + __builtin_ctzll(m); break; }
    }
    int s = first - 1;
    if (s < 0) s = 0;
    if (s >= K) s = K - 1;
    const uint32_t lo = cdf_at(s), hi = cdf_at(s + 1);
    dec_advance(st, RCB_P, lo, hi - lo, in, nw);
    if (lane == 0) {
        out_syms[b] = s;
        states[b] = st;
    }
}

// ================================================================================================
// Compaction: exclusive scan of stream sizes (one workgroup) + gather into a contiguous payload.

// Fused-quantiser tables for parity tests: one wavefront per row.
__global__ void __launch_bounds__(256) k_xq_cdf(const float* __restrict__ logits, int64_t rows, int V, int P,
                                               uint32_t* __restrict__ cdf) {
    const int lane = threadIdx.x & 63;
    const int64_t r = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (r >= rows) return;
    const float* row = logits + r * V;
    float l[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) l[j] = (4 * lane + j < V) ? row[4 * lane + j] : 0.0f;
    XQ q;
    xq_build(q, make_float4(l[0], l[1], l[2], l[3]), lane, V, P);
    uint32_t c = q.base;
    uint32_t* out = cdf + r * (V + 1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k = 4 * lane + j;
        if (k < V) out[k] = xq_cdf_at(q, c, k);
        c += q.f[j];
    }
    if (lane == 0) out[V] = 1u << P;
}

// ================================================================================================
// Host side

static hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

extern "C" int rc_encode_tables(int32_t precision, int32_t cdf_bytes, const void* d_cdf, int32_t K,
                                const uint8_t* d_syms, int32_t streams, int32_t len, uint32_t* d_words,
                                int64_t pitch_words, int32_t* d_nwords, void* stream) {
    if (!d_cdf || !d_syms || !d_words || !d_nwords || streams < 0 || len < 0 || K < 2 || K > 256 ||
        pitch_words < 1)
        return boa_fail(BOA_ERR_ARG, "rc_encode_tables: bad arguments");
    if (streams == 0) return BOA_OK;
    const dim3 grid((streams + 255) / 256), block(256);
    hipStream_t s = as_stream(stream);
    // full tables, whole 16-symbol blocks, 16-byte aligned symbol rows: the pipelined encoder
    if (K == 256 && len >= 16 && len % 16 == 0 && ((uintptr_t)d_syms & 15) == 0 && (precision == 16 || cdf_bytes == 4)) {
        constexpr int R = ENC_LANES_PER_STREAM;
        const dim3 g16((unsigned)(((int64_t)streams * R + 63) / 64)), b16(64);
        if (cdf_bytes == 2 && precision == 16)
            hipLaunchKernelGGL((k_rc_encode_tables16<16, uint16_t, R>), g16, b16, 0, s, (const uint16_t*)d_cdf, d_syms,
                               streams, len, d_words, pitch_words, d_nwords);
        else if (cdf_bytes == 4 && precision == 16)
            hipLaunchKernelGGL((k_rc_encode_tables16<16, uint32_t, R>), g16, b16, 0, s, (const uint32_t*)d_cdf, d_syms,
                               streams, len, d_words, pitch_words, d_nwords);
        else if (cdf_bytes == 4 && precision == 24)
            hipLaunchKernelGGL((k_rc_encode_tables16<24, uint32_t, R>), g16, b16, 0, s, (const uint32_t*)d_cdf, d_syms,
                               streams, len, d_words, pitch_words, d_nwords);
        else
            return boa_fail(BOA_ERR_ARG, "rc_encode_tables: precision %d with %d-byte tables unsupported",
                            precision, cdf_bytes);
        BOA_HIP_TRY(hipGetLastError());
        return BOA_OK;
    }
    if (precision == 16 && cdf_bytes == 2)
        hipLaunchKernelGGL((k_rc_encode_tables<16, uint16_t>), grid, block, 0, s, (const uint16_t*)d_cdf, K,
                           d_syms, streams, len, d_words, pitch_words, d_nwords);
    else if (precision == 16 && cdf_bytes == 4)
        hipLaunchKernelGGL((k_rc_encode_tables<16, uint32_t>), grid, block, 0, s, (const uint32_t*)d_cdf, K,
                           d_syms, streams, len, d_words, pitch_words, d_nwords);
    else if (precision == 24 && cdf_bytes == 4)
        hipLaunchKernelGGL((k_rc_encode_tables<24, uint32_t>), grid, block, 0, s, (const uint32_t*)d_cdf, K,
                           d_syms, streams, len, d_words, pitch_words, d_nwords);
    else
        return boa_fail(BOA_ERR_ARG, "rc_encode_tables: precision %d with %d-byte tables unsupported",
                        precision, cdf_bytes);
    BOA_HIP_TRY(hipGetLastError());
    return BOA_OK;
}

extern "C" int rc_decode_tables(int32_t precision, int32_t cdf_bytes, const void* d_cdf, int32_t K,
                                const uint32_t* d_words, int64_t pitch_words, const int32_t* d_nwords,
                                int32_t streams, int32_t len, uint8_t* d_syms, void* stream) {
    if (!d_cdf || !d_syms || !d_words || !d_nwords || streams < 0 || len < 0 || K < 2 || K > 256 ||
        pitch_words < 1)
        return boa_fail(BOA_ERR_ARG, "rc_decode_tables: bad arguments");
    if (streams == 0) return BOA_OK;
    const dim3 grid(streams), block(64);
    hipStream_t s = as_stream(stream);
    // Full tables, lengths in whole groups of 4 steps, 16-byte aligned tables and 4-byte aligned symbol rows, and
    // sizes whose byte offsets fit the kernels' 32-bit buffer offsets: the throughput decoders (eight streams
    // per wavefront for 2-byte tables at P = 16 and lengths in whole groups of 8 steps, four otherwise).
    const int64_t words_bytes = (int64_t)streams * pitch_words * 4;
    const bool fits = words_bytes < (1ll << 32) - 16 && (int64_t)(streams + 1) * len < (1ll << 32) - 16 &&
                      (int64_t)len * K * cdf_bytes * 4 < (1ll << 31);
    if (K == 256 && len >= 4 && len % 4 == 0 && ((uintptr_t)d_cdf & 15) == 0 && ((uintptr_t)d_syms & 3) == 0 &&
        fits) {
        const dim3 g4((unsigned)((streams + 15) / 16)), b4(256);
        const uint32_t wb = (uint32_t)words_bytes;
        if (cdf_bytes == 2 && precision == 16 && len % 8 == 0 && ((uintptr_t)d_syms & 7) == 0)
            hipLaunchKernelGGL((k_rc_decode_tables8<8>), dim3((unsigned)((streams + 31) / 32)), b4, 0, s,
                               (const uint16_t*)d_cdf, d_words, pitch_words, d_nwords, streams, len, d_syms, wb);
        else if (cdf_bytes == 2 && precision == 16)
            hipLaunchKernelGGL((k_rc_decode_tables4<16, uint16_t>), g4, b4, 0, s, (const uint16_t*)d_cdf, d_words,
                               pitch_words, d_nwords, streams, len, d_syms, wb);
        else if (cdf_bytes == 4 && precision == 16)
            hipLaunchKernelGGL((k_rc_decode_tables4<16, uint32_t>), g4, b4, 0, s, (const uint32_t*)d_cdf, d_words,
                               pitch_words, d_nwords, streams, len, d_syms, wb);
        else if (cdf_bytes == 4 && precision == 24)
            hipLaunchKernelGGL((k_rc_decode_tables4<24, uint32_t>), g4, b4, 0, s, (const uint32_t*)d_cdf, d_words,
                               pitch_words, d_nwords, streams, len, d_syms, wb);
        else
            return boa_fail(BOA_ERR_ARG, "rc_decode_tables: precision %d with %d-byte tables unsupported",
                            precision, cdf_bytes);
        BOA_HIP_TRY(hipGetLastError());
        return BOA_OK;
    }
    if (precision == 16 && cdf_bytes == 2)
        hipLaunchKernelGGL((k_rc_decode_tables<16, uint16_t>), grid, block, 0, s, (const uint16_t*)d_cdf, K,
                           d_words, pitch_words, d_nwords, streams, len, d_syms);
    else if (precision == 16 && cdf_bytes == 4)
        hipLaunchKernelGGL((k_rc_decode_tables<16, uint32_t>), grid, block, 0, s, (const uint32_t*)d_cdf, K,
                           d_words, pitch_words, d_nwords, streams, len, d_syms);
    else if (precision == 24 && cdf_bytes == 4)
        hipLaunchKernelGGL((k_rc_decode_tables<24, uint32_t>), grid, block, 0, s, (const uint32_t*)d_cdf, K,
                           d_words, pitch_words, d_nwords, streams, len, d_syms);
    else
        return boa_fail(BOA_ERR_ARG, "rc_decode_tables: precision %d with %d-byte tables unsupported",
                        precision, cdf_bytes);
    BOA_HIP_TRY(hipGetLastError());
    return BOA_OK;
}

extern "C" int rc_synth_tables(uint64_t seed, float sigma, int32_t precision, int32_t cdf_bytes, int32_t K,
                               int32_t streams, int32_t len, void* d_cdf, uint8_t* d_syms, void* stream) {
    if (!d_cdf || !d_syms || streams < 0 || len < 0 || K < 2 || K > 256)
        return boa_fail(BOA_ERR_ARG, "rc_synth_tables: bad arguments");
    const int64_t rows = (int64_t)streams * len;
    if (rows == 0) return BOA_OK;
    const int64_t waves = rows < (int64_t)65536 * 4 ? rows : (int64_t)65536 * 4;
    const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
    hipStream_t s = as_stream(stream);
    if (precision == 16 && cdf_bytes == 2)
        hipLaunchKernelGGL((k_rc_synth_tables<16, uint16_t>), grid, block, 0, s, seed, sigma, K, streams, len,
                           (uint16_t*)d_cdf, d_syms);
    else if (precision == 16 && cdf_bytes == 4)
        hipLaunchKernelGGL((k_rc_synth_tables<16, uint32_t>), grid, block, 0, s, seed, sigma, K, streams, len,
                           (uint32_t*)d_cdf, d_syms);
    else if (precision == 24 && cdf_bytes == 4)
        hipLaunchKernelGGL((k_rc_synth_tables<24, uint32_t>), grid, block, 0, s, seed, sigma, K, streams, len,
                           (uint32_t*)d_cdf, d_syms);
    else
        return boa_fail(BOA_ERR_ARG, "rc_synth_tables: precision %d with %d-byte tables unsupported",
                        precision, cdf_bytes);
    BOA_HIP_TRY(hipGetLastError());
    return BOA_OK;
}

extern "C" int boa_xq_cdf(const float* d_logits, int64_t rows, int32_t vocab, int32_t precision,
                          uint32_t* d_cdf, void* stream) {
    if (!d_logits || !d_cdf || rows < 0 || vocab < 2 || vocab > 256 || precision < 16 || precision > 24)
        return boa_fail(BOA_ERR_ARG, "boa_xq_cdf: bad arguments");
    if (rows == 0) return BOA_OK;
    const int64_t blocks = (rows + 3) / 4;
    hipLaunchKernelGGL(k_xq_cdf, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), d_logits, rows, vocab,
                       precision, d_cdf);
    BOA_HIP_TRY(hipGetLastError());
    return BOA_OK;
}

// ------------------------------------------------------------------------------------------------
// RangeCoderBatch holder (gpu_range_coder.py:212-306): owns states, the pitched word buffer and sizes.
struct rcb {
    int32_t n = 0, k = 0;
    int64_t pitch = 0;
    hipStream_t stream = nullptr;
    EncState* enc = nullptr;
    DecState* dec = nullptr;
    uint32_t* words = nullptr;
    int32_t* sizes = nullptr;
    int64_t* off = nullptr;
    uint32_t* payload = nullptr;
    bool finalized = false;
    bool dec_ready = false;
};

extern "C" int rcb_destroy(rcb* b) {
    if (!b) return BOA_OK;
    if (b->stream) (void)hipStreamSynchronize(b->stream);
    else (void)hipDeviceSynchronize();
    void* ptrs[] = {b->enc, b->dec, b->words, b->sizes, b->off, b->payload};
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
    delete b;
    return BOA_OK;
}

extern "C" int rcb_create(int32_t n, int32_t k, int64_t pitch_words, void* stream, rcb** out) {
    if (!out || n < 1 || k < 1 || k > RCB_KMAX || pitch_words < 1)
        return boa_fail(BOA_ERR_ARG, "rcb_create: need N >= 1, 1 <= K <= %d, pitch >= 1 (got %d, %d, %lld)",
                        RCB_KMAX, n, k, (long long)pitch_words);
    *out = nullptr;
    rcb* b = new rcb();
    b->n = n;
    b->k = k;
    b->pitch = pitch_words;
    b->stream = as_stream(stream);
    hipError_t e = hipSuccess;
    if (e == hipSuccess) e = hipMalloc((void**)&b->enc, sizeof(EncState) * n);
    if (e == hipSuccess) e = hipMalloc((void**)&b->dec, sizeof(DecState) * n);
    if (e == hipSuccess) e = hipMalloc((void**)&b->words, sizeof(uint32_t) * (size_t)n * (size_t)pitch_words);
    if (e == hipSuccess) e = hipMalloc((void**)&b->sizes, sizeof(int32_t) * n);
    if (e == hipSuccess) e = hipMalloc((void**)&b->off, sizeof(int64_t) * n);
    if (e == hipSuccess) e = hipMemsetAsync(b->sizes, 0, sizeof(int32_t) * n, b->stream);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(k_rcb_init, dim3((n + 255) / 256), dim3(256), 0, b->stream, b->enc, n);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(b->stream);
    if (e != hipSuccess) {
        rcb_destroy(b);
        return boa_fail_hip(e, "rcb_create", __FILE__, __LINE__);
    }
    *out = b;
    return BOA_OK;
}

extern "C" int rcb_encode_step(rcb* b, const int32_t* d_syms, const float* d_probs, const uint8_t* d_mask) {
    if (!b || !d_syms || !d_probs) return boa_fail(BOA_ERR_ARG, "rcb_encode_step: null argument");
    if (b->finalized) return boa_fail(BOA_ERR_STATE, "rcb_encode_step: batch already finalized");
    hipLaunchKernelGGL(k_rcb_encode_step, dim3(b->n), dim3(64), 0, b->stream, d_syms, d_probs, d_mask, b->n, b->k,
                       b->enc, b->words, b->pitch);
    BOA_HIP_TRY(hipGetLastError());
    return BOA_OK;
}

extern "C" int rcb_finalize(rcb* b) {
    if (!b) return boa_fail(BOA_ERR_ARG, "rcb_finalize: null batch");
    hipLaunchKernelGGL(k_rcb_finalize, dim3((b->n + 255) / 256), dim3(256), 0, b->stream, b->enc, b->words, b->pitch,
                       b->sizes, b->n);
    BOA_HIP_TRY(hipGetLastError());
    b->finalized = true;
    std::vector<int32_t> h(b->n);
    BOA_HIP_TRY(hipMemcpyAsync(h.data(), b->sizes, sizeof(int32_t) * b->n, hipMemcpyDeviceToHost, b->stream));
    BOA_HIP_TRY(hipStreamSynchronize(b->stream));
    for (int i = 0; i < b->n; ++i)
        if (h[i] < 0)
            return boa_fail(BOA_ERR_OVERFLOW, "Compressed stream %d needs %d words, exceeds pitch %lld; increase pitch",
                            i, -h[i], (long long)b->pitch);
    return BOA_OK;
}

extern "C" int rcb_get_sizes(rcb* b, int32_t* h_sizes) {
    if (!b || !h_sizes) return boa_fail(BOA_ERR_ARG, "rcb_get_sizes: null argument");
    BOA_HIP_TRY(hipMemcpyAsync(h_sizes, b->sizes, sizeof(int32_t) * b->n, hipMemcpyDeviceToHost, b->stream));
    BOA_HIP_TRY(hipStreamSynchronize(b->stream));
    return BOA_OK;
}

extern "C" int rcb_get_words(rcb* b, uint32_t* h_words, int64_t cap_words, int64_t* h_total) {
    if (!b || !h_total) return boa_fail(BOA_ERR_ARG, "rcb_get_words: null argument");
    int64_t total = 0;
    // the compacted payload is at most n * pitch words; gather into a scratch buffer owned by the batch
    if (!b->payload) BOA_HIP_TRY(hipMalloc((void**)&b->payload, sizeof(uint32_t) * (size_t)b->n * (size_t)b->pitch));
    int rc = boa_compact(b->words, b->pitch, b->sizes, b->n, b->off, b->payload, (int64_t)b->n * b->pitch, &total,
                         b->stream);
    if (rc != BOA_OK) return rc;
    *h_total = total;
    if (total > cap_words) return boa_fail(BOA_ERR_OVERFLOW, "rcb_get_words: host buffer too small");
    if (total > 0) {
        if (!h_words) return boa_fail(BOA_ERR_ARG, "rcb_get_words: null host buffer");
        BOA_HIP_TRY(hipMemcpyAsync(h_words, b->payload, sizeof(uint32_t) * total, hipMemcpyDeviceToHost, b->stream));
    }
    BOA_HIP_TRY(hipStreamSynchronize(b->stream));
    return BOA_OK;
}

extern "C" int rcb_load(rcb* b, const uint32_t* h_words, const int32_t* h_sizes) {
    if (!b || !h_sizes) return boa_fail(BOA_ERR_ARG, "rcb_load: null argument");
    std::vector<uint32_t> buf((size_t)b->n * (size_t)b->pitch, 0u);
    int64_t pos = 0;
    for (int i = 0; i < b->n; ++i) {
        const int32_t nw = h_sizes[i];
        if (nw < 0) return boa_fail(BOA_ERR_ARG, "rcb_load: negative size for stream %d", i);
        if (nw > b->pitch) return boa_fail(BOA_ERR_OVERFLOW, "Compressed stream exceeds pitch; increase pitch");
        if (nw > 0) memcpy(buf.data() + (size_t)i * (size_t)b->pitch, h_words + pos, sizeof(uint32_t) * nw);
        pos += nw;
    }
    BOA_HIP_TRY(hipMemcpyAsync(b->words, buf.data(), sizeof(uint32_t) * buf.size(), hipMemcpyHostToDevice, b->stream));
    BOA_HIP_TRY(hipMemcpyAsync(b->sizes, h_sizes, sizeof(int32_t) * b->n, hipMemcpyHostToDevice, b->stream));
    BOA_HIP_TRY(hipStreamSynchronize(b->stream));
    b->dec_ready = false;
    return BOA_OK;
}

extern "C" int rcb_init_decoder(rcb* b) {
    if (!b) return boa_fail(BOA_ERR_ARG, "rcb_init_decoder: null batch");
    hipLaunchKernelGGL(k_rcb_init_dec, dim3((b->n + 255) / 256), dim3(256), 0, b->stream, b->dec, b->words, b->pitch,
                       b->sizes, b->n);
    BOA_HIP_TRY(hipGetLastError());
    b->dec_ready = true;
    return BOA_OK;
}

extern "C" int rcb_decode_step(rcb* b, const float* d_probs, int32_t* d_out_syms, const uint8_t* d_mask) {
    if (!b || !d_probs || !d_out_syms) return boa_fail(BOA_ERR_ARG, "rcb_decode_step: null argument");
    if (!b->dec_ready) return boa_fail(BOA_ERR_STATE, "rcb_decode_step: call init_decoder first");
    hipLaunchKernelGGL(k_rcb_decode_step, dim3(b->n), dim3(64), 0, b->stream, d_probs, d_mask, b->n, b->k, b->dec,
                       b->words, b->pitch, b->sizes, d_out_syms);
    BOA_HIP_TRY(hipGetLastError());
    return BOA_OK;
}
