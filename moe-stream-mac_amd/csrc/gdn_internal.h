// Launch-level interface between the C ABI (gdn_api.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace gdn {

struct RecFwdArgs {
    const void *q, *k, *v;
    const float *g, *beta, *state0;
    const uint8_t *mask;
    void *y;
    float *state_T, *snaps;
    int B, T, Hk, Hv, Dk, Dv, chunk, in_dt, out_dt, gate;
};

struct RecBwdArgs {
    const void *q, *k, *v;
    const float *g, *beta, *state0;
    const uint8_t *mask;
    const float *snaps;
    const void *dy;
    const float *dstate_T;
    void *dq, *dk, *dv;
    float *dg, *dbeta, *dstate0;
    float *ws_sub;   // sub-chunk start states, per workgroup
    float *part_qk;  // [nrb][B][T][Hv][2][Dk] per-row-block dq | dk
    float *part_gb;  // [nrb][B][T][Hv][2]     per-row-block dbeta | dg
    float *part_gv;  // [nrb][B][T][Hv][Dk]    per-row-block dg (vector gate)
    int B, T, Hk, Hv, Dk, Dv, chunk, in_dt, dy_dt, grad_dt, gate, nrb, max_sub;
};

// Chunked (WY/UT) form, C = 64, Dk = Dv = 128 (gdn_chunk.hip).
struct ChunkSizes {
    size_t H, G, T, P, W, U, Dl, saved;  // offsets into / size of the buffer kept from forward to backward
    size_t dH, dDl, part, work;          // offsets into / size of the backward workspace
};
ChunkSizes chunk_sizes(int B, int T, int Hv);

struct ChunkCall {
    const void *q, *k, *v;
    const float *g, *beta, *state0;
    const void *dy;
    const float *dstate_T;
    void *y, *dv;
    float *state_T, *dg, *dbeta, *dstate0;
    void *saved, *work;
    int B, T, Hk, Hv, in_dt, out_dt, dy_dt, grad_dt, gate;
};
// stage: "prep" | "fwd" (forward) or "seq" | "local" (backward)
void launch_chunk_stage(const ChunkCall &cc, const char *stage, hipStream_t st);

int pick_lane_width(int Dk);
int rec_num_row_blocks(int Dv);
int rec_max_sub(int T, int chunk);
size_t rec_sub_floats(int B, int Hv, int Dk, int Dv, int T, int chunk);

void launch_rec_fwd(const RecFwdArgs &a, hipStream_t st);
void launch_rec_bwd(const RecBwdArgs &a, hipStream_t st);
void launch_rec_bwd_reduce(const RecBwdArgs &a, hipStream_t st);
void launch_reduce_qk(const RecBwdArgs &a, hipStream_t st);
void launch_copy_or_zero(float *dst, const float *src, size_t n, hipStream_t st);

}  // namespace gdn
