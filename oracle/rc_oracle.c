/*
 * oracle/rc_oracle.c -- CPU restatement of the reference's range coder and CDF quantisers.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (boa-constrictor_amd/) links, loads or calls this
 * file; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the checker.
 *
 * What is restated, and from where (paths are into the reference checkout):
 *   - encoder state / encode step      gpu_range_coder.py:42-48, 88-141   (same in range_coder_kernels.cu:38-102)
 *   - finalize                         gpu_range_coder.py:143-168         (range_coder_kernels.cu:271-300)
 *   - decoder init / decode step       gpu_range_coder.py:170-210         (range_coder_kernels.cu:311-327)
 *   - Q2 quantiser build_cdf_fast      gpu_range_coder.py:57-79           (range_coder_kernels.cu:10-32)
 *   - XQ quantiser: this build's own fused quantiser (no reference counterpart; see ora_xq_cdf).
 *   - ora_expf: this build's own exp (Cody-Waite reduction + Taylor polynomial), the same algorithm the
 *     GPU kernels use inside the XQ quantiser, so the CPU reproduces GPU tables bit for bit.
 *
 * Build with -ffp-contract=off (oracle/Makefile): every float/double operation below must round exactly
 * once, as written, so that results are reproducible op-for-op.
 *
 * Pinning (tests/test_oracle_rc.py): an independent big-integer interval checker (oracle/bigint_check.py),
 * hand-derived known answers (tests/golden/rc_known_answers.json), closed forms (empty stream -> 0 words,
 * uniform Q2 table), code-length bounds and round trips.
 */
#include <stdint.h>
#include <stddef.h>
#include <string.h>
#include <math.h>

typedef struct {
    uint64_t lower;
    uint64_t range;
    int32_t inverted_num;
    uint32_t first_inv_lower_word;
    int64_t nwords;   /* words produced so far (may exceed cap: then the output is truncated) */
} ora_enc;

typedef struct {
    uint64_t lower;
    uint64_t range;
    uint64_t point;
    int64_t read_idx;
} ora_dec;

static void emit(ora_enc* st, uint32_t w, uint32_t* out, int64_t cap) {
    if (st->nwords < cap) out[st->nwords] = w;
    st->nwords++;
}

void ora_enc_init(ora_enc* st) {
    st->lower = 0ull;
    st->range = 0xFFFFFFFFFFFFFFFFull;
    st->inverted_num = 0;
    st->first_inv_lower_word = 0u;
    st->nwords = 0;
}

/* gpu_range_coder.py:100-140 */
void ora_enc_push(ora_enc* st, int P, uint32_t left, uint32_t prob, uint32_t* out, int64_t cap) {
    uint64_t scale = st->range >> P;
    st->range = scale * (uint64_t)prob;
    uint64_t old_lower = st->lower;
    st->lower = st->lower + scale * (uint64_t)left;
    if (st->inverted_num > 0) {
        uint64_t sum = st->lower + st->range;
        if (sum > st->lower) {
            uint32_t first_word, subsequent;
            if (st->lower < old_lower) { first_word = st->first_inv_lower_word + 1u; subsequent = 0u; }
            else { first_word = st->first_inv_lower_word; subsequent = 0xFFFFFFFFu; }
            emit(st, first_word, out, cap);
            for (int i = 1; i < st->inverted_num; ++i) emit(st, subsequent, out, cap);
            st->inverted_num = 0;
        }
    }
    while (st->range < (1ull << 32)) {
        uint32_t lower_word = (uint32_t)(st->lower >> 32);
        st->lower <<= 32;
        st->range <<= 32;
        if (st->inverted_num > 0) {
            if (st->inverted_num < 0x7FFFFFFF) st->inverted_num += 1;
        } else {
            uint64_t sum = st->lower + st->range;
            if (sum > st->lower) {
                emit(st, lower_word, out, cap);
            } else {
                st->inverted_num = 1;
                st->first_inv_lower_word = lower_word;
            }
        }
    }
}

/* gpu_range_coder.py:143-168; returns the total word count */
int64_t ora_enc_finish(ora_enc* st, uint32_t* out, int64_t cap) {
    if (st->range == 0xFFFFFFFFFFFFFFFFull) return st->nwords; /* empty stream */
    uint64_t point = st->lower + ((1ull << 32) - 1ull);
    if (st->inverted_num > 0) {
        uint32_t first_word, subsequent;
        if (point < st->lower) { first_word = st->first_inv_lower_word + 1u; subsequent = 0u; }
        else { first_word = st->first_inv_lower_word; subsequent = 0xFFFFFFFFu; }
        emit(st, first_word, out, cap);
        for (int i = 1; i < st->inverted_num; ++i) emit(st, subsequent, out, cap);
        st->inverted_num = 0;
    }
    uint32_t point_word = (uint32_t)(point >> 32);
    emit(st, point_word, out, cap);
    uint64_t upper = st->lower + st->range;
    uint32_t upper_word = (uint32_t)(upper >> 32);
    if (upper_word == point_word) emit(st, 0u, out, cap);
    return st->nwords;
}

static uint32_t next_word(ora_dec* st, const uint32_t* in, int64_t n) {
    return (st->read_idx < n) ? in[st->read_idx++] : 0u;
}

/* gpu_range_coder.py:170-180 */
void ora_dec_init(ora_dec* st, const uint32_t* in, int64_t n) {
    st->lower = 0ull; st->range = 0xFFFFFFFFFFFFFFFFull; st->point = 0ull; st->read_idx = 0;
    for (int i = 0; i < 2; ++i) st->point = (st->point << 32) | (uint64_t)next_word(st, in, n);
}

/* gpu_range_coder.py:191-194: the quantile the next symbol is looked up with */
uint32_t ora_dec_target(const ora_dec* st, int P) {
    uint64_t scale = st->range >> P;
    uint64_t q = (st->point - st->lower) / scale;
    if (q >= (1ull << P)) q = (1ull << P) - 1ull;
    return (uint32_t)q;
}

/* gpu_range_coder.py:196-198: smallest k+1 with cdf[k+1] > target, minus one (linear, as written) */
int ora_find_symbol(const uint32_t* cdf, int K, uint32_t target) {
    int next_symbol = 1;
    while (next_symbol <= K && !(cdf[next_symbol] > target)) ++next_symbol;
    int s = next_symbol - 1;
    if (s < 0) s = 0;
    if (s >= K) s = K - 1;
    return s;
}

/* gpu_range_coder.py:200-209 */
void ora_dec_advance(ora_dec* st, int P, uint32_t left, uint32_t prob, const uint32_t* in, int64_t n) {
    uint64_t scale = st->range >> P;
    st->lower = st->lower + scale * (uint64_t)left;
    st->range = scale * (uint64_t)prob;
    while (st->range < (1ull << 32)) {
        st->lower <<= 32;
        st->range <<= 32;
        st->point = (st->point << 32) | (uint64_t)next_word(st, in, n);
    }
}

/* ---------------------------------------------------------------------------------------------- */
/* Q2: gpu_range_coder.py:57-79 (build_cdf_fast), sequential double accumulation, cdf has K+1 entries */
void ora_q2_cdf(const float* probs, int K, int P, uint32_t* cdf) {
    const uint32_t TOTAL = 1u << P;
    if (K <= 0) { cdf[0] = 0; cdf[1] = TOTAL; return; }
    const uint32_t free_weight = TOTAL - (uint32_t)K;
    double norm = 0.0;
    for (int i = 0; i < K; ++i) norm += (double)probs[i];
    if (!(norm > 0.0) || !isfinite(norm)) {
        uint32_t acc = 0;
        for (int i = 0; i < K; ++i) { cdf[i] = acc; acc += (free_weight / (uint32_t)K) + 1u; }
        cdf[K] = TOTAL;
        return;
    }
    double scale = (double)free_weight / norm;
    double cumulative_float = 0.0;
    uint32_t accumulated_slack = 0;
    for (int i = 0; i < K; ++i) {
        cdf[i] = (uint32_t)(cumulative_float * scale) + accumulated_slack;
        cumulative_float += (double)probs[i];
        accumulated_slack += 1u;
    }
    cdf[K] = TOTAL;
}

/* ---------------------------------------------------------------------------------------------- */
/* This build's exp: Cody & Waite (1980) argument reduction x = k*ln2 + r, |r| <= ln2/2, then the degree-7
 * Taylor polynomial of e^r in Horner form, then scaling by 2^k.  ln2 is split into a head with 16
 * significant bits (so k*LN2_HI is exact for |k| < 256) and a tail.  Every operation is a single IEEE
 * binary32 operation; the GPU kernels (csrc/boa_common.h: boa_expf) perform the same sequence. */
#define ORA_LN2_HI 0x1.62e4p-1f             /* 0.693145751953125 (16 significant bits) */
#define ORA_LN2_LO 0x1.7f7d1cp-20f          /* ln2 - LN2_HI rounded to binary32 */
#define ORA_LOG2E 0x1.715476p+0f            /* 1/ln2 rounded to binary32 */

float ora_expf(float x) {
    if (!(x >= -87.0f)) return 0.0f;          /* also maps NaN to 0 */
    if (x > 88.0f) x = 88.0f;
    float kf = rintf(x * ORA_LOG2E);
    float r = x - kf * ORA_LN2_HI;
    r = r - kf * ORA_LN2_LO;
    float p = 0x1.a01a02p-13f;                /* 1/7! */
    p = p * r + 0x1.6c16c2p-10f;              /* 1/6! */
    p = p * r + 0x1.111112p-7f;               /* 1/5! */
    p = p * r + 0x1.555556p-5f;               /* 1/4! */
    p = p * r + 0x1.555556p-3f;               /* 1/3! */
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return ldexpf(p, (int)kf);
}

/* XQ quantiser (this build's fused CDF; no reference counterpart).  Same outer form as Q2
 * (cdf[i] = floor(cum_i * free / norm) + i, cdf[K] = 2^P) but the cumulative sums are exact integers, so a
 * wavefront prefix sum reproduces them in any order:
 *   m = max_i l_i;  e_i = ora_expf(l_i - m);  f_i = trunc(e_i * 2^23)  (f_argmax = 2^23)
 *   c_i = sum_{j<i} f_j (exact);  S = c_K;  inv = (double)(2^P - K) / (double)S
 *   cdf_i = (uint32)((double)c_i * inv) + i   (i < K),   cdf_K = 2^P
 * If S == 0 (all logits NaN) the Q2 uniform fallback is used. */
void ora_xq_cdf(const float* logits, int K, int P, uint32_t* cdf) {
    const uint32_t TOTAL = 1u << P;
    const uint32_t free_weight = TOTAL - (uint32_t)K;
    float m = -INFINITY;
    for (int i = 0; i < K; ++i) m = fmaxf(m, logits[i]);
    uint32_t f[1024];
    uint64_t S = 0;
    for (int i = 0; i < K; ++i) {
        float e = ora_expf(logits[i] - m);
        f[i] = (uint32_t)(e * 8388608.0f);
        S += f[i];
    }
    if (S == 0) {
        uint32_t acc = 0;
        for (int i = 0; i < K; ++i) { cdf[i] = acc; acc += (free_weight / (uint32_t)K) + 1u; }
        cdf[K] = TOTAL;
        return;
    }
    double inv = (double)free_weight / (double)S;
    uint64_t c = 0;
    for (int i = 0; i < K; ++i) {
        cdf[i] = (uint32_t)((double)c * inv) + (uint32_t)i;
        c += f[i];
    }
    cdf[K] = TOTAL;
}

/* ---------------------------------------------------------------------------------------------- */
/* Whole-stream helpers (one stream = one chunk lane).  Tables: [T][K+1] uint32. */
int64_t ora_encode_tables(int P, const uint32_t* cdf, int K, const int32_t* syms, int64_t T,
                          uint32_t* out, int64_t cap) {
    ora_enc st; ora_enc_init(&st);
    for (int64_t t = 0; t < T; ++t) {
        const uint32_t* c = cdf + t * (int64_t)(K + 1);
        int s = syms[t];
        if (s < 0 || s >= K) continue;   /* gpu_range_coder.py:97: invalid symbols are skipped */
        ora_enc_push(&st, P, c[s], c[s + 1] - c[s], out, cap);
    }
    return ora_enc_finish(&st, out, cap);
}

void ora_decode_tables(int P, const uint32_t* cdf, int K, int64_t T, const uint32_t* in, int64_t n,
                       int32_t* syms) {
    ora_dec st; ora_dec_init(&st, in, n);
    for (int64_t t = 0; t < T; ++t) {
        const uint32_t* c = cdf + t * (int64_t)(K + 1);
        uint32_t q = ora_dec_target(&st, P);
        int s = ora_find_symbol(c, K, q);
        syms[t] = s;
        ora_dec_advance(&st, P, c[s], c[s + 1] - c[s], in, n);
    }
}

/* Per-step Q2 from probabilities (the reference RangeCoderBatch semantics for one lane): probs [T][K] */
int64_t ora_encode_probs_q2(int P, const float* probs, int K, const int32_t* syms, int64_t T,
                            uint32_t* out, int64_t cap) {
    uint32_t cdf[1025];
    ora_enc st; ora_enc_init(&st);
    for (int64_t t = 0; t < T; ++t) {
        int s = syms[t];
        if (s < 0 || s >= K) continue;
        ora_q2_cdf(probs + t * (int64_t)K, K, P, cdf);
        ora_enc_push(&st, P, cdf[s], cdf[s + 1] - cdf[s], out, cap);
    }
    return ora_enc_finish(&st, out, cap);
}

void ora_decode_probs_q2(int P, const float* probs, int K, int64_t T, const uint32_t* in, int64_t n,
                         int32_t* syms) {
    uint32_t cdf[1025];
    ora_dec st; ora_dec_init(&st, in, n);
    for (int64_t t = 0; t < T; ++t) {
        ora_q2_cdf(probs + t * (int64_t)K, K, P, cdf);
        uint32_t q = ora_dec_target(&st, P);
        int s = ora_find_symbol(cdf, K, q);
        syms[t] = s;
        ora_dec_advance(&st, P, cdf[s], cdf[s + 1] - cdf[s], in, n);
    }
}

/* Per-step XQ from logits: logits [T][K] */
int64_t ora_encode_logits_xq(int P, const float* logits, int K, const int32_t* syms, int64_t T,
                             uint32_t* out, int64_t cap) {
    uint32_t cdf[1025];
    ora_enc st; ora_enc_init(&st);
    for (int64_t t = 0; t < T; ++t) {
        int s = syms[t];
        if (s < 0 || s >= K) continue;
        ora_xq_cdf(logits + t * (int64_t)K, K, P, cdf);
        ora_enc_push(&st, P, cdf[s], cdf[s + 1] - cdf[s], out, cap);
    }
    return ora_enc_finish(&st, out, cap);
}

void ora_decode_logits_xq(int P, const float* logits, int K, int64_t T, const uint32_t* in, int64_t n,
                          int32_t* syms) {
    uint32_t cdf[1025];
    ora_dec st; ora_dec_init(&st, in, n);
    for (int64_t t = 0; t < T; ++t) {
        ora_xq_cdf(logits + t * (int64_t)K, K, P, cdf);
        uint32_t q = ora_dec_target(&st, P);
        int s = ora_find_symbol(cdf, K, q);
        syms[t] = s;
        ora_dec_advance(&st, P, cdf[s], cdf[s + 1] - cdf[s], in, n);
    }
}

/* Batched table builders (numpy convenience): rows x K -> rows x (K+1) */
void ora_q2_cdf_rows(const float* probs, int64_t rows, int K, int P, uint32_t* cdf) {
    for (int64_t r = 0; r < rows; ++r) ora_q2_cdf(probs + r * K, K, P, cdf + r * (int64_t)(K + 1));
}

void ora_xq_cdf_rows(const float* logits, int64_t rows, int K, int P, uint32_t* cdf) {
    for (int64_t r = 0; r < rows; ++r) ora_xq_cdf(logits + r * K, K, P, cdf + r * (int64_t)(K + 1));
}

void ora_expf_rows(const float* x, int64_t n, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = ora_expf(x[i]);
}

/* ---------------------------------------------------------------------------------------------- */
/* Per-lane incremental calls, one symbol at a time (the CPU baseline calls these once per lane per step,
 * as codec.py:201 calls constriction's encoder once per lane per step). */
size_t ora_enc_sizeof(void) { return sizeof(ora_enc); }
size_t ora_dec_sizeof(void) { return sizeof(ora_dec); }

void ora_q2_encode_one(ora_enc* st, int P, const float* probs, int K, int sym, uint32_t* out, int64_t cap) {
    uint32_t cdf[1025];
    if (sym < 0 || sym >= K) return;
    ora_q2_cdf(probs, K, P, cdf);
    ora_enc_push(st, P, cdf[sym], cdf[sym + 1] - cdf[sym], out, cap);
}

int ora_q2_decode_one(ora_dec* st, int P, const float* probs, int K, const uint32_t* in, int64_t n) {
    uint32_t cdf[1025];
    ora_q2_cdf(probs, K, P, cdf);
    int s = ora_find_symbol(cdf, K, ora_dec_target(st, P));
    ora_dec_advance(st, P, cdf[s], cdf[s + 1] - cdf[s], in, n);
    return s;
}
