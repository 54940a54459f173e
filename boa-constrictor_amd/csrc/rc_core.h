// Range-coder core of libboa_hip.so: the integer algorithm of gpu_range_coder.py:88-210 (u64 state, u32
// words, PRECISION P), as functions over a register-resident state.  Included by boa_common.h for the
// kernels (BOA_HD = __host__ __device__ __forceinline__) and by the CPU check of this exact code
// (tests/native/coder_host_check.cpp, BOA_HD = inline), which compares it with exact 64-bit division and
// with the oracle's coder under the address and undefined-behaviour sanitizers.
#pragma once

#include <stdint.h>

#ifndef BOA_HD
#define BOA_HD inline
#endif

namespace boa {

// Words are emitted through a bounds-checked sink; overflow is recorded instead of writing past the pitch.
struct EncState {
    uint64_t lower;
    uint64_t range;
    int32_t inverted_num;
    uint32_t first_inv_lower_word;
    int32_t nwords;
    int32_t overflow;
};

struct DecState {
    uint64_t lower;
    uint64_t range;
    uint64_t point;
    int32_t read_idx;
    int32_t pad;
};

BOA_HD void enc_init(EncState& st) {
    st.lower = 0ull;
    st.range = 0xFFFFFFFFFFFFFFFFull;
    st.inverted_num = 0;
    st.first_inv_lower_word = 0u;
    st.nwords = 0;
    st.overflow = 0;
}

// Word sink: only the designated writer lane stores; every lane keeps the same counters.
struct WordSink {
    uint32_t* out;
    int64_t cap;
    bool writer;
    BOA_HD void put(EncState& st, uint32_t w) const {
        if (st.nwords < cap) {
            if (writer) out[st.nwords] = w;
        } else {
            st.overflow = 1;
        }
        st.nwords++;
    }
};

// gpu_range_coder.py:100-140.  A zero width (only possible with an invalid table) is clamped to 1 as
// range_coder_kernels.cu:558,698-700 does; with valid tables (freq >= 1) this changes nothing.  The
// renormalisation loop runs at most twice: for P <= 32 a valid step needs at most one shift.
BOA_HD void enc_push(EncState& st, int P, uint32_t left, uint32_t prob, const WordSink& sink) {
    if (prob == 0u) prob = 1u;
    const uint64_t scale = st.range >> P;
    st.range = scale * (uint64_t)prob;
    const uint64_t old_lower = st.lower;
    st.lower = st.lower + scale * (uint64_t)left;
    if (st.inverted_num > 0) {
        const uint64_t sum = st.lower + st.range;
        if (sum > st.lower) {
            uint32_t first_word, subsequent;
            if (st.lower < old_lower) { first_word = st.first_inv_lower_word + 1u; subsequent = 0u; }
            else { first_word = st.first_inv_lower_word; subsequent = 0xFFFFFFFFu; }
            sink.put(st, first_word);
            for (int i = 1; i < st.inverted_num; ++i) sink.put(st, subsequent);
            st.inverted_num = 0;
        }
    }
    for (int it = 0; it < 2 && st.range < (1ull << 32); ++it) {
        const uint32_t lower_word = (uint32_t)(st.lower >> 32);
        st.lower <<= 32;
        st.range <<= 32;
        if (st.inverted_num > 0) {
            if (st.inverted_num < 0x7FFFFFFF) st.inverted_num += 1;
        } else {
            const uint64_t sum = st.lower + st.range;
            if (sum > st.lower) sink.put(st, lower_word);
            else { st.inverted_num = 1; st.first_inv_lower_word = lower_word; }
        }
    }
}

// gpu_range_coder.py:143-168
BOA_HD void enc_finish(EncState& st, const WordSink& sink) {
    if (st.range == 0xFFFFFFFFFFFFFFFFull) return;  // nothing encoded: empty stream
    const uint64_t point = st.lower + ((1ull << 32) - 1ull);
    if (st.inverted_num > 0) {
        uint32_t first_word, subsequent;
        if (point < st.lower) { first_word = st.first_inv_lower_word + 1u; subsequent = 0u; }
        else { first_word = st.first_inv_lower_word; subsequent = 0xFFFFFFFFu; }
        sink.put(st, first_word);
        for (int i = 1; i < st.inverted_num; ++i) sink.put(st, subsequent);
        st.inverted_num = 0;
    }
    const uint32_t point_word = (uint32_t)(point >> 32);
    sink.put(st, point_word);
    const uint64_t upper = st.lower + st.range;
    if ((uint32_t)(upper >> 32) == point_word) sink.put(st, 0u);
}

// gpu_range_coder.py:170-180
BOA_HD void dec_init(DecState& st, const uint32_t* in, int32_t n) {
    st.lower = 0ull; st.range = 0xFFFFFFFFFFFFFFFFull; st.point = 0ull; st.read_idx = 0; st.pad = 0;
    for (int i = 0; i < 2; ++i) {
        const uint32_t w = (st.read_idx < n) ? in[st.read_idx++] : 0u;
        st.point = (st.point << 32) | (uint64_t)w;
    }
}

// gpu_range_coder.py:191-194: q = min(floor((point - lower) / scale), 2^P - 1), scale = range >> P.
// The exact u64 quotient is obtained without a 64-bit integer division: an fp64 quotient estimate (relative
// error ~2^-52, so below 1 in absolute terms for q <= 2^P) clamped to [0, 2^P], then one integer
// correction step.  q_est * scale cannot overflow: q_est <= 2^P and scale < 2^(64 - P).
BOA_HD uint32_t dec_target(const DecState& st, int P) {
    const uint64_t scale = st.range >> P;
    if (scale == 0ull) return 0u;
    const uint64_t d = st.point - st.lower;
    const uint64_t cap = 1ull << P;
    const double qd = (double)d / (double)scale;
    uint64_t q = qd >= (double)cap ? cap : (uint64_t)qd;
    const uint64_t prod = q * scale;
    if (prod > d) q -= 1ull;                      // estimate one too high
    else if (d - prod >= scale && q < cap) q += 1ull;  // estimate one too low
    if (q >= cap) q = cap - 1ull;
    return (uint32_t)q;
}

// The same quotient for P <= 16 from an fp32 estimate: d and scale rounded to fp32 (each within 2^-23
// relative, as hi * 2^32 + lo with two roundings), their quotient within about 2^-21 relative (the device
// reciprocal adds 1 ulp), i.e. below 2^-5 in absolute terms for q <= 2^16; then dec_target's clamp and one-step
// integer correction, which make it exact.  Branch-free (scale = 0 gives 0, as dec_target).
BOA_HD float u64_to_f32(uint64_t v) {
    uint32_t hi = (uint32_t)(v >> 32), lo = (uint32_t)v;
#ifdef __HIP_DEVICE_COMPILE__
    __asm__("" : "+v"(hi));  // two 32-bit conversions, not the compiler's exactly rounded 64-bit sequence
#endif
    return (float)hi * 4294967296.0f + (float)lo;
}
BOA_HD uint32_t dec_target16(const DecState& st, int P) {
    const uint64_t scale = st.range >> P;
    const uint64_t sc = scale ? scale : 1ull;
    const uint64_t d = st.point - st.lower;
    const uint32_t cap = 1u << P;
#ifdef __HIP_DEVICE_COMPILE__
    const float qf = u64_to_f32(d) * __builtin_amdgcn_rcpf(u64_to_f32(sc));
#else
    const float qf = u64_to_f32(d) / u64_to_f32(sc);
#endif
    uint32_t q = qf >= (float)cap ? cap : (uint32_t)qf;
    const uint64_t prod = (uint64_t)q * sc;
    q = prod > d ? q - 1u : ((d - prod >= sc && q < cap) ? q + 1u : q);
    q = q >= cap ? cap - 1u : q;
    return scale ? q : 0u;
}

// gpu_range_coder.py:200-209
BOA_HD void dec_advance(DecState& st, int P, uint32_t left, uint32_t prob,
                                            const uint32_t* in, int32_t n) {
    if (prob == 0u) prob = 1u;
    const uint64_t scale = st.range >> P;
    st.lower = st.lower + scale * (uint64_t)left;
    st.range = scale * (uint64_t)prob;
    for (int it = 0; it < 2 && st.range < (1ull << 32); ++it) {
        st.lower <<= 32;
        st.range <<= 32;
        const uint32_t w = (st.read_idx < n) ? in[st.read_idx++] : 0u;
        st.point = (st.point << 32) | (uint64_t)w;
    }
}

}  // namespace boa
