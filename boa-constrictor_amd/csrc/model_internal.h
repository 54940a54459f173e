// Host/device interface between the model context (model.hip) and the fused decompress-step kernels
// (fused_step.hip for d_model 256, fused_step512.hip for d_model 512).  Internal to libboa_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "boa_common.h"

namespace boa {

// Fragment-packed bfloat16 GEMM weights for MFMA 16x16x32 B operands: matrix W [N][K] (N % 16 == 0,
// K % 32 == 0) as blocks (f, s) for f < N/16, s < K/32, in order f-major; a block is 64 lanes x 8 values,
// lane l holding W[16f + (l % 16)][32s + 8(l / 16) + j], j < 8: the hi part, then (bf16x3) the lo part.
// One wavefront reads a block with one fully coalesced 16-byte load per lane.
struct FusedLayer {
    const float *ln1_w, *ln1_b, *in_b, *conv_w, *conv_b, *dt_w, *dt_b, *Aneg, *D, *out_b, *ln2_w, *ln2_b, *ff1_b,
        *ff2_b;
    const uint16_t *in_p, *x_p, *out_p, *ff1_p, *ff2_p;
};

// The layer table as the d_model 256 fused kernel reads it: constant memory (the table does not change while the
// kernel runs), so its pointers come through scalar loads, which wait on the scalar counter alone.  Read as global
// memory, each pointer is a vector load, and the wait for it is also a wait for every vector load and store
// issued before it (the counter is in order): at a phase boundary, the previous phase's state stores.  (The
// d_model 512 kernel, short of scalar registers, measured 4.5% slower with it and reads the table as global
// memory.)
typedef __attribute__((address_space(4))) const FusedLayer CFusedLayer;
__device__ __forceinline__ CFusedLayer& layer_at(const FusedLayer* table, int l) {
    return ((CFusedLayer*)table)[l];
}

struct FusedArgs {
    const FusedLayer* layers;  // device array [L]
    int L;
    int V;
    int B;                     // lanes in this launch
    int p0m3;                  // absolute position of this step, mod 3 (conv history ring slot)
    int64_t max_lanes;         // lane capacity of the state arrays
    const float *emb, *h1_b, *h2_b;
    const uint16_t *h1_p, *h2_p;
    float* ssm;                // [L][max_lanes][NS/4][di][4]
    float* hist;               // [L][max_lanes][3][di]
    const int32_t* tokens_in;  // [B] model input bytes
    float* logits;             // [B][V] output, or null
    // decode steps (decode != 0): positions t .. t + nsteps - 1, each step's symbol fed back as the next
    // step's input; the last one is left in tokens_out.  Without decode, nsteps must be 1.
    int decode;
    int t;
    int nsteps;
    int stagger_us;            // start offset between workgroup classes (multi-step launches), microseconds
    int stagger_classes;       // number of classes (1, 2, 4 or 8 sets of XCDs)
    const int32_t* lens;
    DecState* dec;
    const uint32_t* payload;
    int64_t payload_words;     // the payload's length: every lane's stream is clamped to it
    const int64_t* off;
    const int32_t* nwords;
    int32_t* tokens_out;
    uint8_t* out;
    int64_t out_stride;
    // d_model 512 kernel only: per-lane scratch in device memory (the context's workspace rows, row = lane): the
    // mixer's z | conv output [lanes][2 d_inner]
    float* scr;
};

// Supported shape of the fused kernel: d_model 256, d_state 16, dt_rank 16, d_conv 4, vocab % 16 == 0.
bool fused_step_supported(int d_model, int d_state, int dt_rank, int d_conv, int vocab);

// nt = 3 (bf16x3 weights, hi + lo) or 2 (bf16 weights); 512 threads per workgroup of 16 lanes
hipError_t launch_fused_step(const FusedArgs& a, int nt, hipStream_t s);

// The d_model 512 form (d_inner 1024, d_state 16, dt_rank 32, d_conv 4, vocab 256): 512 threads (8 waves) per
// workgroup of 32 lanes, one workgroup per CU (256 VGPRs per thread, 145 KB of LDS with the residual stream).
bool fused_step512_supported(int d_model, int d_state, int dt_rank, int d_conv, int vocab);
hipError_t launch_fused_step512(const FusedArgs& a, int nt, hipStream_t s);

}  // namespace boa
