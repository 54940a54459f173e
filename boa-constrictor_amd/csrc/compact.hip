// Bitstream compaction: the pitched per-lane word buffers of a wave become the contiguous BOA2 payload
// (every chunk's words back to back, boa.py:239-248), with each lane's word offset.
//
// Reference: the reference copies the whole pitch of every lane to the host and slices there
// (gpu_range_coder.py:278-292; boa.cpp:388-395).  Here the offsets are an exclusive prefix sum of the
// word counts computed on the device by a three-kernel multi-workgroup scan (no atomics, so the result
// does not depend on scheduling), then one workgroup per lane gathers its words.  Only the payload's
// total crosses to the host.
//
// The scan keeps one partial sum per workgroup of 1024 lanes plus the total in a scratch buffer:
//   boa_compact          a buffer the library allocates once per device and stream (and grows when a
//                        larger wave arrives), kept until the process ends;
//   boa_compact_noalloc  the file-scope device array `scratch` (at most kMaxScanBlocks workgroups, i.e.
//                        262144 lanes), for callers that cannot allocate; every call on one GPU shares it,
//                        so calls that overlap on one GPU race.
#include "boa_common.h"

#include <map>
#include <mutex>
#include <utility>

#include "../../include/boa_hip.h"

using namespace boa;

namespace {
constexpr int kScanBlockLanes = 1024;  // lanes per scan workgroup
constexpr int kStaticScanBlocks = BOA_COMPACT_NOALLOC_MAX_LANES / kScanBlockLanes;  // partials the static array holds
static_assert(kStaticScanBlocks * kScanBlockLanes == BOA_COMPACT_NOALLOC_MAX_LANES, "static scratch size");
}  // namespace

// boa_compact_noalloc's scratch: [0] = total words, [1 + w] = partial of scan workgroup w.  Nothing in it
// needs clearing between calls: every call writes each entry before it reads it.
static __device__ __align__(256) int64_t scratch[1 + kStaticScanBlocks];

namespace {

constexpr int kScanBlock = kScanBlockLanes;
constexpr int kMaxScanBlocks = kStaticScanBlocks;  // also the smallest allocation of boa_compact's scratch
constexpr int kMaxDevices = 64;

// A lane's word count must lie in [0, pitch].  An invalid one counts as 0 words and marks its scan workgroup's
// partial with kBadBlock, which the one-workgroup scan turns into a negative total: the host then reports the
// error and launches no gather (which would read past the lane's row).
constexpr int64_t kBadBlock = -1;

__device__ __forceinline__ int64_t lane_words(const int32_t* nwords, int n, int64_t pitch, int i, int& bad) {
    if (i >= n) return 0;
    const int32_t w = nwords[i];
    bad = (w < 0 || w > pitch) ? 1 : 0;
    return bad ? (int64_t)0 : (int64_t)w;
}

// Inclusive prefix sum over a 1024-thread workgroup (16 wavefronts): wavefront shuffles, then the 16
// wavefront totals scanned by the first wavefront through LDS.  Integer adds: exact in any order.
__device__ __forceinline__ int64_t block_incl_scan(int64_t v, int64_t* sw) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int64_t t = __shfl_up(v, o, 64);
        if (lane >= o) v += t;
    }
    if (lane == 63) sw[wave] = v;
    __syncthreads();
    if (wave == 0) {
        int64_t w = lane < kScanBlock / 64 ? sw[lane] : 0;
#pragma unroll
        for (int o = 1; o < kScanBlock / 64; o <<= 1) {
            const int64_t t = __shfl_up(w, o, 64);
            if (lane >= o) w += t;
        }
        if (lane < kScanBlock / 64) sw[lane] = w;
    }
    __syncthreads();
    return wave ? v + sw[wave - 1] : v;
}

// Kernel 1: sums[w] = words of lanes [1024 w, 1024 w + 1024), or kBadBlock if one of them has an invalid count.
__global__ void __launch_bounds__(kScanBlock) k_block_sums(const int32_t* __restrict__ nwords, int n, int64_t pitch,
                                                          int64_t* __restrict__ sums) {
    __shared__ int64_t sw[kScanBlock / 64];
    const int i = blockIdx.x * kScanBlock + threadIdx.x;
    int bad = 0;
    const int64_t incl = block_incl_scan(lane_words(nwords, n, pitch, i, bad), sw);
    const int any_bad = __syncthreads_or(bad);
    if (threadIdx.x == kScanBlock - 1) sums[blockIdx.x] = any_bad ? kBadBlock : incl;
}

// Kernel 2 (one workgroup): sums[0..nb) -> exclusive prefix sums in place; *total = their sum, or kBadBlock if
// any partial is.  Each thread takes a contiguous run of ceil(nb / 1024) entries.
__global__ void __launch_bounds__(kScanBlock) k_scan_block_sums(int64_t* __restrict__ sums, int nb,
                                                               int64_t* __restrict__ total) {
    __shared__ int64_t sw[kScanBlock / 64];
    const int per = (nb + kScanBlock - 1) / kScanBlock;
    const int lo = threadIdx.x * per, hi = min(nb, lo + per);
    int64_t s = 0;
    int bad = 0;
    for (int i = lo; i < hi; ++i) {
        const int64_t v = sums[i];
        bad |= v < 0 ? 1 : 0;
        s += v;
    }
    const int any_bad = __syncthreads_or(bad);
    int64_t run = block_incl_scan(s, sw) - s;
    for (int i = lo; i < hi; ++i) {
        const int64_t v = sums[i];
        sums[i] = run;
        run += v;
    }
    if (threadIdx.x == kScanBlock - 1) *total = any_bad ? kBadBlock : run;
}

// Kernel 3: off[i] = exclusive prefix of the words of lanes < i (meaningless when the total is kBadBlock).
__global__ void __launch_bounds__(kScanBlock) k_lane_offsets(const int32_t* __restrict__ nwords, int n, int64_t pitch,
                                                            const int64_t* __restrict__ sums,
                                                            int64_t* __restrict__ off) {
    __shared__ int64_t sw[kScanBlock / 64];
    const int i = blockIdx.x * kScanBlock + threadIdx.x;
    int bad = 0;
    const int64_t v = lane_words(nwords, n, pitch, i, bad);
    const int64_t incl = block_incl_scan(v, sw);
    if (i < n) off[i] = sums[blockIdx.x] + incl - v;
}

// One workgroup per lane copies its words to its offset.
__global__ void __launch_bounds__(256) k_gather_words(const uint32_t* __restrict__ words, int64_t pitch,
                                                     const int32_t* __restrict__ nwords,
                                                     const int64_t* __restrict__ off,
                                                     uint32_t* __restrict__ payload) {
    const int b = blockIdx.x;
    const int64_t nw = min((int64_t)max(nwords[b], 0), pitch);  // counts are checked before this launch
    const uint32_t* src = words + (int64_t)b * pitch;
    uint32_t* dst = payload + off[b];
    for (int i = threadIdx.x; i < nw; i += blockDim.x) dst[i] = src[i];
}

int scan_blocks(int32_t lanes) { return (lanes + kScanBlock - 1) / kScanBlock; }

// Scan, total to the host, capacity check, gather.  sc: 1 + scan_blocks(lanes) int64 of device scratch:
// [0] = total words, [1 + w] = exclusive offset of scan workgroup w (its partial sum before the scan).
int compact_with(const char* who, int64_t* sc, const uint32_t* d_words, int64_t pitch_words, const int32_t* d_nwords,
                 int32_t lanes, int64_t* d_word_off, uint32_t* d_payload, int64_t payload_cap, int64_t* h_total,
                 hipStream_t s) {
    const int nb = scan_blocks(lanes);
    hipLaunchKernelGGL(k_block_sums, dim3(nb), dim3(kScanBlock), 0, s, d_nwords, lanes, pitch_words, sc + 1);
    hipLaunchKernelGGL(k_scan_block_sums, dim3(1), dim3(kScanBlock), 0, s, sc + 1, nb, sc);
    hipLaunchKernelGGL(k_lane_offsets, dim3(nb), dim3(kScanBlock), 0, s, d_nwords, lanes, pitch_words, sc + 1,
                       d_word_off);
    BOA_HIP_TRY(hipGetLastError());
    int64_t total = 0;
    BOA_HIP_TRY(hipMemcpyAsync(&total, sc, sizeof(int64_t), hipMemcpyDeviceToHost, s));
    BOA_HIP_TRY(hipStreamSynchronize(s));
    if (total < 0) {
        *h_total = 0;
        return boa_fail(BOA_ERR_ARG, "%s: a lane's word count lies outside [0, pitch_words = %lld]", who,
                        (long long)pitch_words);
    }
    *h_total = total;
    if (total > payload_cap)
        return boa_fail(BOA_ERR_OVERFLOW, "%s: payload needs %lld words, capacity %lld", who, (long long)total,
                        (long long)payload_cap);
    if (total > 0) {
        if (!d_payload) return boa_fail(BOA_ERR_ARG, "%s: null payload", who);
        hipLaunchKernelGGL(k_gather_words, dim3(lanes), dim3(256), 0, s, d_words, pitch_words, d_nwords, d_word_off,
                           d_payload);
        BOA_HIP_TRY(hipGetLastError());
    }
    BOA_HIP_TRY(hipStreamSynchronize(s));
    return BOA_OK;
}

std::mutex g_mu;
struct HeapScratch {
    int64_t* p = nullptr;
    int64_t cap = 0;  // int64 entries
};
std::map<std::pair<int, hipStream_t>, HeapScratch> g_heap;  // boa_compact's scratch, per (device, stream)

int64_t* g_static[kMaxDevices] = {};  // device address of `scratch`, per device

int current_device(const char* who, int* dev) {
    BOA_HIP_TRY(hipGetDevice(dev));
    if (*dev < 0 || *dev >= kMaxDevices) return boa_fail(BOA_ERR_ARG, "%s: device %d out of range", who, *dev);
    return BOA_OK;
}

}  // namespace

extern "C" int boa_compact(const uint32_t* d_words, int64_t pitch_words, const int32_t* d_nwords, int32_t lanes,
                           int64_t* d_word_off, uint32_t* d_payload, int64_t payload_cap, int64_t* h_total_words,
                           void* stream) {
    if (!d_words || !d_nwords || !d_word_off || lanes < 0 || pitch_words < 0 || !h_total_words)
        return boa_fail(BOA_ERR_ARG, "boa_compact: bad arguments");
    *h_total_words = 0;
    if (lanes == 0) return BOA_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    int dev = 0;
    int rc = current_device("boa_compact", &dev);
    if (rc != BOA_OK) return rc;
    const int64_t need = 1 + scan_blocks(lanes);
    int64_t* sc = nullptr;
    {
        // allocated on the first call per (device, stream) and when a wave needs more partials than before;
        // calls on one stream are ordered by it, so they may share the buffer; the previous buffer is freed
        // only after the stream has finished with it
        std::lock_guard<std::mutex> g(g_mu);
        HeapScratch& h = g_heap[std::make_pair(dev, s)];
        if (h.cap < need) {
            if (h.p) {
                BOA_HIP_TRY(hipStreamSynchronize(s));
                (void)hipFree(h.p);
                h.p = nullptr;
                h.cap = 0;
            }
            const int64_t cap = need < 1 + kMaxScanBlocks ? 1 + kMaxScanBlocks : need;
            BOA_HIP_TRY(hipMalloc((void**)&h.p, sizeof(int64_t) * (size_t)cap));
            h.cap = cap;
        }
        sc = h.p;
    }
    return compact_with("boa_compact", sc, d_words, pitch_words, d_nwords, lanes, d_word_off, d_payload, payload_cap,
                        h_total_words, s);
}

extern "C" int boa_compact_noalloc(const uint32_t* d_words, int64_t pitch_words, const int32_t* d_nwords,
                                   int32_t lanes, int64_t* d_word_off, uint32_t* d_payload, int64_t payload_cap,
                                   int64_t* h_total_words, void* stream) {
    if (!d_words || !d_nwords || !d_word_off || lanes < 0 || pitch_words < 0 || !h_total_words)
        return boa_fail(BOA_ERR_ARG, "boa_compact_noalloc: bad arguments");
    *h_total_words = 0;
    if (lanes > BOA_COMPACT_NOALLOC_MAX_LANES)
        return boa_fail(BOA_ERR_ARG, "boa_compact_noalloc: %d lanes exceed the static scratch maximum of %d", lanes,
                        BOA_COMPACT_NOALLOC_MAX_LANES);
    if (lanes == 0) return BOA_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    int dev = 0;
    int rc = current_device("boa_compact_noalloc", &dev);
    if (rc != BOA_OK) return rc;
    int64_t* sc = nullptr;
    {
        // the array's own name is a host-side stand-in: its device address (one copy per GPU) is looked up
        // once per device and used for every kernel argument and copy
        std::lock_guard<std::mutex> g(g_mu);
        if (!g_static[dev]) {
            void* p = nullptr;
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return boa_fail_hip(e, "hipGetSymbolAddress(scratch)", __FILE__, __LINE__);
            if (!p) return boa_fail(BOA_ERR_HIP, "boa_compact_noalloc: scratch has no device address");
            g_static[dev] = static_cast<int64_t*>(p);
        }
        sc = g_static[dev];
    }
    return compact_with("boa_compact_noalloc", sc, d_words, pitch_words, d_nwords, lanes, d_word_off, d_payload,
                        payload_cap, h_total_words, s);
}
