// CPU check of the product range-coder core (boa-constrictor_amd/csrc/rc_core.h, the exact code the kernels
// run), built with g++ under AddressSanitizer and UndefinedBehaviorSanitizer by tests/test_coder_host.py.
//   1. dec_target (fp64 quotient estimate + one integer correction), and at P = 16 dec_target16 (fp32
//      estimate + the same correction), equal the exact u64 quotient
//      min((point - lower) / (range >> P), 2^P - 1) of gpu_range_coder.py:191-194 on random decoder states,
//      on corrupt-stream states (point - lower anywhere in [0, 2^64)), and on boundary states (scale 2^8,
//      d at and next to multiples of scale, d near 2^P * scale, the largest d and range);
//   2. enc_push / enc_finish produce the same words as the oracle's restatement (oracle/rc_oracle.c) on
//      random and skewed tables (long carry runs), and dec_init / dec_target / dec_advance decode them back;
//   3. a word sink whose capacity is too small records the overflow and writes nothing past its end.
// Exit status 0 when every check holds; the first failure is printed.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "rc_core.h"

extern "C" {
int64_t ora_encode_tables(int P, const uint32_t* cdf, int K, const int32_t* syms, int64_t T, uint32_t* out,
                          int64_t cap);
}

namespace {

uint64_t g_rng = 0x9E3779B97F4A7C15ull;
uint64_t next64() {  // splitmix64
    uint64_t z = (g_rng += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

int fails = 0;
long long checked_targets = 0;

void check_target(uint64_t lower, uint64_t range, uint64_t point, int P) {
    boa::DecState st{};
    st.lower = lower;
    st.range = range;
    st.point = point;
    const uint64_t scale = range >> P;
    uint64_t q = (point - lower) / scale;
    if (q >= (1ull << P)) q = (1ull << P) - 1ull;
    const uint32_t got = boa::dec_target(st, P);
    ++checked_targets;
    if (got != (uint32_t)q && fails++ < 5)
        std::printf("dec_target mismatch P=%d lower=%llu range=%llu point=%llu: got %u want %llu\n", P,
                    (unsigned long long)lower, (unsigned long long)range, (unsigned long long)point, got,
                    (unsigned long long)q);
    if (P <= 16) {
        const uint32_t g16 = boa::dec_target16(st, P);
        if (g16 != (uint32_t)q && fails++ < 5)
            std::printf("dec_target16 mismatch P=%d lower=%llu range=%llu point=%llu: got %u want %llu\n", P,
                        (unsigned long long)lower, (unsigned long long)range, (unsigned long long)point, g16,
                        (unsigned long long)q);
    }
}

void targets() {
    const int Ps[2] = {16, 24};
    for (int P : Ps) {
        // random valid decoder states: range in [2^32, 2^64), point - lower below range
        for (int i = 0; i < 2000000; ++i) {
            const uint64_t range = (next64() | (1ull << 32)) >> (next64() % 32);
            const uint64_t r = range < (1ull << 32) ? (1ull << 32) : range;
            const uint64_t lower = next64();
            check_target(lower, r, lower + next64() % r, P);
        }
        // corrupt streams: point anywhere
        for (int i = 0; i < 1000000; ++i) {
            const uint64_t r = (next64() | (1ull << 32));
            check_target(next64(), r >> (next64() % 32 == 0 ? 0 : (next64() % 32)) | (1ull << 32), next64(), P);
        }
        // boundaries: smallest scale (range = 2^32), d at and around multiples of scale and at the cap
        const uint64_t ranges[4] = {1ull << 32, (1ull << 32) + 1, ~0ull, (1ull << 63)};
        for (uint64_t r : ranges) {
            const uint64_t scale = r >> P;
            for (uint64_t k : {0ull, 1ull, 2ull, 255ull, (1ull << P) - 2, (1ull << P) - 1, 1ull << P,
                               (1ull << P) + 1, ~0ull / scale}) {
                for (int64_t delta = -2; delta <= 2; ++delta) {
                    const uint64_t d = k * scale + (uint64_t)delta;
                    check_target(0, r, d, P);
                    check_target(0x8000000000000000ull, r, 0x8000000000000000ull + d, P);
                }
            }
            check_target(0, r, ~0ull, P);
            check_target(1, r, 0, P);  // point below lower: wraps to 2^64 - 1
        }
    }
}

// Table with K entries cdf[0..K] (cdf[K] = 2^P), every frequency >= 1; skew > 0 gives one symbol almost all
// of the mass.
void make_table(int K, int P, int skew, uint32_t* cdf) {
    const uint32_t total = 1u << P;
    std::vector<uint32_t> f(K, 1u);
    uint32_t left = total - (uint32_t)K;
    if (skew) {
        f[(int)(next64() % K)] += left;
    } else {
        for (int i = 0; i < K && left; ++i) {
            const uint32_t take = (i == K - 1) ? left : (uint32_t)(next64() % (left + 1) / 2);
            f[i] += take;
            left -= take;
        }
        f[K - 1] += left;
    }
    cdf[0] = 0;
    for (int i = 0; i < K; ++i) cdf[i + 1] = cdf[i] + f[i];
}

void round_trips() {
    const int Ps[2] = {16, 24};
    for (int trial = 0; trial < 400; ++trial) {
        const int P = Ps[trial & 1];
        const int K = 2 + (int)(next64() % 255);
        const int T = 1 + (int)(next64() % 1500);
        const int skew = (trial % 3 == 0);
        std::vector<uint32_t> cdf((size_t)T * (K + 1));
        std::vector<int32_t> syms(T);
        for (int t = 0; t < T; ++t) {
            uint32_t* c = &cdf[(size_t)t * (K + 1)];
            make_table(K, P, skew, c);
            // draw the symbol from the table (inverse CDF of a uniform P-bit value); skewed tables
            // sometimes force the rare symbols, which makes carry runs
            const uint32_t u = (uint32_t)(next64() & ((1ull << P) - 1));
            int s = 0;
            while (s + 1 < K && c[s + 1] <= u) ++s;
            if (skew && next64() % 7 == 0) s = (int)(next64() % K);
            syms[t] = s;
        }
        const int64_t cap = T + 8;
        std::vector<uint32_t> want(cap), got(cap + 16, 0xDEADBEEFu);
        const int64_t nw = ora_encode_tables(P, cdf.data(), K, syms.data(), T, want.data(), cap);
        boa::EncState st;
        boa::enc_init(st);
        const boa::WordSink sink{got.data(), cap, true};
        for (int t = 0; t < T; ++t) {
            const uint32_t* c = &cdf[(size_t)t * (K + 1)];
            boa::enc_push(st, P, c[syms[t]], c[syms[t] + 1] - c[syms[t]], sink);
        }
        boa::enc_finish(st, sink);
        if (st.nwords != nw || st.overflow || std::memcmp(got.data(), want.data(), sizeof(uint32_t) * nw) != 0) {
            if (fails++ < 5) std::printf("encoder words differ from the oracle (trial %d, P=%d K=%d T=%d)\n", trial, P, K, T);
            continue;
        }
        if (got[cap] != 0xDEADBEEFu && fails++ < 5) std::printf("encoder wrote past its capacity\n");
        boa::DecState ds;
        boa::dec_init(ds, got.data(), (int32_t)nw);
        for (int t = 0; t < T; ++t) {
            const uint32_t* c = &cdf[(size_t)t * (K + 1)];
            const uint32_t q = boa::dec_target(ds, P);
            int s = 0;
            while (s + 1 < K && c[s + 1] <= q) ++s;
            if (s != syms[t]) {
                if (fails++ < 5) std::printf("decode mismatch trial %d t %d: %d vs %d\n", trial, t, s, syms[t]);
                break;
            }
            boa::dec_advance(ds, P, c[s], c[s + 1] - c[s], got.data(), (int32_t)nw);
        }
        // the same stream into a sink that is too small: overflow is recorded, nothing is written past it
        if (nw > 2) {
            const int64_t small = nw / 2;
            std::vector<uint32_t> buf(small);
            boa::EncState s2;
            boa::enc_init(s2);
            const boa::WordSink tiny{buf.data(), small, true};
            for (int t = 0; t < T; ++t) {
                const uint32_t* c = &cdf[(size_t)t * (K + 1)];
                boa::enc_push(s2, P, c[syms[t]], c[syms[t] + 1] - c[syms[t]], tiny);
            }
            boa::enc_finish(s2, tiny);
            if ((!s2.overflow || s2.nwords != nw) && fails++ < 5) std::printf("overflow not recorded\n");
        }
    }
}

}  // namespace

int main() {
    targets();
    round_trips();
    std::printf("dec_target cases %lld, failures %d\n", checked_targets, fails);
    return fails ? 1 : 0;
}
