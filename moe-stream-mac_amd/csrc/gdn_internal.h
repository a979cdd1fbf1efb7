// Launch-level interface between the C ABI (gdn_api.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "gdn_common.h"

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
constexpr int kChunkC = 64;
constexpr int kChunkD = 128;

// Offsets of the per-chunk buffers of one launch covering T tokens of B sequences: the tile set ck_prep and the
// sequential forward write ("saved"; bwd = false leaves out what only the backward reads), and the backward
// workspace.  A zero-sized buffer has no storage.  The fp32 set (bf16 = false) and the bf16 set keep different
// tiles.
struct ChunkSizes {
    struct Buf {
        size_t off, size;
    };
    Buf H, G, T, P, W, U, Dl;         // tile set
    Buf Wb, KTb, Pb, PTb, QTb, nWTb;  // bf16 operand tiles of the bf16 set
    Buf Gv, QGb, KDb;                 // per-channel gates (bf16 set)
    size_t saved;                     // size of the tile set
    Buf dH, dDl, part, vgd;           // backward workspace
    size_t work;                      // its size
};
// vg: the per-channel gate kind (vg_kind), bf16 set only.
ChunkSizes chunk_sizes(int B, int T, int Hk, int Hv, bool bf16, bool bwd, int vg = 0);
// The per-channel gate kind of a gate: 0 one decay per head, 1 per-channel log decays, 2 per-channel decays (whose
// backward also keeps the pieces ck_vg_dg forms d/d(decay) from, in the vgd buffer).
inline int vg_kind(int gate) { return gate == GATE_LOG_VEC ? 1 : gate == GATE_DECAY_VEC ? 2 : 0; }

// One launch of a chunked stage.  q, k, v, g, beta, y, dy, dq, dk, dv, dg and dbeta point at the launch's first
// token; T is the launch's token count and Ts the token stride of a sequence (the full length).  tiles / work are
// the chunk_sizes(B, T, ...) buffers of this launch.
struct ChunkCall {
    const void *q, *k, *v;
    const float *g, *beta, *state0;
    const void *dy;
    const float *dstate_T;
    void *y, *dq, *dk, *dv;
    float *state_T, *dg, *dbeta, *dstate0;
    void *tiles, *work;
    float *snap;        // window snapshots (see ck::Args)
    int wc, win0, recompute, fwd_only;
    int B, T, Ts, Hk, Hv, in_dt, out_dt, dy_dt, grad_dt, gate;
};
// stage: "prep" | "fwd" (forward) or "seq" | "local" (backward; "local" walks the value heads of each key head
// and writes dq and dk).  With recompute, "fwd" runs every window of the launch at once.
void launch_chunk_stage(const ChunkCall &cc, const char *stage, hipStream_t st);
// The chunked form takes per-channel gates (GATE_DECAY_VEC, GATE_LOG_VEC) for bf16 inputs (gdn_chunk_vg.hip).
bool chunk_vg_supported(int in_dt);

// Masked steps on the chunked form (gdn_mask.hip): tensors of B*T tokens, contiguous; q, k [tok][Hk][Dk], v, y, dy
// [tok][Hv][Dv], g, beta [tok][Hv] (the raw gates), mask [tok]; Z, Yp, dy1, dz and the passes' parts fp32.
struct MaskArgs {
    const void *q, *k, *v, *dy;
    const float *g, *beta;
    const uint8_t *mask;
    void *y;          // forward: holds y' on entry, y on exit
    const float *Z;   // second pass output S' k
    float *Yp;        // the first pass's fp32 output y' (read at masked tokens by the backward), or NULL
    float *dy1, *dz;  // cotangents of the two passes
    const float *dq1, *dk1, *dv1, *dg1, *dbeta1, *dq2, *dk2, *dv2, *dg2, *dbeta2;
    void *dq, *dk, *dv;
    float *dg, *dbeta;
    int Hk, Hv, Dk, Dv, in_dt, out_dt, dy_dt, grad_dt, gate;
};
int mask_max_heads();
void launch_mask_gates(const float *g, const float *beta, const uint8_t *mask, float *g2, float *beta2,
                       size_t tokens, int Hv, int gate, hipStream_t st);
void launch_mask_fix_fwd(const MaskArgs &a, size_t tokens, hipStream_t st);
void launch_mask_bwd_cot(const MaskArgs &a, size_t tokens, hipStream_t st);
void launch_mask_bwd_combine(const MaskArgs &a, size_t tokens, hipStream_t st);
void launch_add2(float *dst, const float *x, const float *y, size_t n, hipStream_t st);

int pick_lane_width(int Dk);
int rec_num_row_blocks(int Dv);
int rec_bwd_rows(int B, int Hv, int Dk, int Dv, int gate);
int rec_bwd_row_blocks(int B, int Hv, int Dk, int Dv, int gate);
int rec_max_sub(int T, int chunk);
size_t rec_sub_floats(int B, int Hv, int Dk, int Dv, int T, int chunk, int gate);

void launch_rec_fwd(const RecFwdArgs &a, hipStream_t st);
void launch_rec_decode(const RecFwdArgs &a, hipStream_t st);  // T = 1, no mask, no snapshots
void launch_rec_bwd(const RecBwdArgs &a, hipStream_t st);
void launch_rec_bwd_reduce(const RecBwdArgs &a, hipStream_t st);
void launch_copy_or_zero(float *dst, const float *src, size_t n, hipStream_t st);

// Block ops around the recurrence (gdn_block_ops.hip).  `vec` selects the vector-load kernels; the caller
// checks alignment and shape for them.
int row_lanes(int D);
int gates_max_heads();
int conv_kmax();
int grms_dmax();
size_t gates_bwd_work_floats(size_t tokens, int Hv);
size_t conv_bwd_work_floats(int B, int T, int C, int K);
size_t grms_bwd_work_floats(size_t rows, int D);
void launch_gates_fwd(const void *a, const void *b, const float *A_log, const float *dt_bias, float *g, float *beta,
                      size_t tokens, int Hv, int in_dt, int log_space, float beta_scale, hipStream_t st);
void launch_gates_bwd(const void *a, const void *b, const float *A_log, const float *dt_bias, const float *g,
                      const float *dg, const float *dbeta, void *da, void *db, float *dA_log, float *ddt_bias,
                      float *work, size_t tokens, int Hv, int in_dt, int grad_dt, int log_space, float beta_scale,
                      hipStream_t st);
void launch_l2norm_fwd(const void *x, void *y, size_t rows, int D, float eps, float scale, int dt, bool vec,
                       hipStream_t st);
void launch_l2norm_bwd(const void *x, const void *dy, void *dx, size_t rows, int D, float eps, float scale, int dt,
                       int dy_dt, bool vec, hipStream_t st);
// Conv + SiLU over [B][T][C]; with qk > 0 fused with the q/k/v split ([0,qk) q, [qk,2qk) k, rest v) and the
// per-head L2 norm of q (times scale_q) and k.  Forward: q/k/v are outputs (qk = 0: v is the [B][T][C] output).
// Backward: q/k/v are the cotangents (dtype g_dt), dx/dw the results, work the dw partials.
struct ConvCall {
    const void *x;
    const float *w, *state_in;
    void *q, *k, *v;
    float *state_out;
    void *dx;
    float *dw, *work;
    int B, T, C, K, qk, Dk, dt, g_dt;
    float scale_q, eps;
    bool vec;
};
bool conv_qkv_supported(int Dk, int K, int dt, int g_dt, bool vec, int C);
void launch_conv_fwd(const ConvCall &c, hipStream_t st);
void launch_conv_bwd(const ConvCall &c, hipStream_t st);
void launch_grms_fwd(const void *y, const void *z, const float *w, void *out, size_t rows, int D, float eps, int dt,
                     int z_dt, bool vec, hipStream_t st);
void launch_grms_bwd(const void *y, const void *z, const float *w, const void *dout, void *dy, void *dz, float *dw,
                     float *work, size_t rows, int D, float eps, int dt, int z_dt, int dout_dt, bool vec,
                     hipStream_t st);

}  // namespace gdn
