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

int pick_lane_width(int Dk);
int rec_num_row_blocks(int Dv);
int rec_max_sub(int T, int chunk);
size_t rec_sub_floats(int B, int Hv, int Dk, int Dv, int T, int chunk);

void launch_rec_fwd(const RecFwdArgs &a, hipStream_t st);
void launch_rec_bwd(const RecBwdArgs &a, hipStream_t st);
void launch_rec_bwd_reduce(const RecBwdArgs &a, hipStream_t st);
void launch_copy_or_zero(float *dst, const float *src, size_t n, hipStream_t st);

}  // namespace gdn
