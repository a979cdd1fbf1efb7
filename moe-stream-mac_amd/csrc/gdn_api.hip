// C ABI of the GDN engine (declared in include/gdn_mi355x.h): argument checks, workspace layout, dispatch.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <mutex>
#include <algorithm>
#include <atomic>
#include <string>
#include <type_traits>
#include <vector>

#include "gdn_common.h"
#include "gdn_internal.h"
#include "../../include/gdn_mi355x.h"

namespace gdn {

static thread_local char g_err[512];

static int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

static bool debug_sync() {
    static const int on = [] {
        const char *s = getenv("GDN_DEBUG_SYNC");
        return s && s[0] == '1';
    }();
    return on != 0;
}

// After a launch: report launch errors, and in debug mode synchronise and report execution errors.
static int check_launch(hipStream_t st, const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
    if (debug_sync()) {
        e = hipStreamSynchronize(st);
        if (e != hipSuccess) return fail(GDN_ERR_LAUNCH, "%s: execution failed: %s", what, hipGetErrorString(e));
    }
    return GDN_OK;
}

// Opt-in launch timing (gdn_profile_enable): each launch is bracketed by two HIP events recorded on the
// launch's own stream.  Off by default; the normal path records nothing.
struct ProfRec {
    const char *name;
    hipEvent_t start, stop;
};
static std::mutex g_prof_mu;
static std::vector<ProfRec> g_prof;
static std::atomic<bool> g_prof_on{false};  // read by every launch without the lock

struct Timed {
    const char *name;
    hipStream_t st;
    hipEvent_t start = nullptr, stop = nullptr;
    Timed(const char *n, hipStream_t s) : name(n), st(s) {
        if (!g_prof_on.load(std::memory_order_relaxed)) return;
        if (hipEventCreate(&start) != hipSuccess || hipEventCreate(&stop) != hipSuccess) {
            start = stop = nullptr;
            return;
        }
        (void)hipEventRecord(start, st);
    }
    ~Timed() {
        if (!start) return;
        (void)hipEventRecord(stop, st);
        std::lock_guard<std::mutex> lk(g_prof_mu);
        g_prof.push_back({name, start, stop});
    }
};

__global__ void copy_or_zero_kernel(float *dst, const float *src, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = src ? src[i] : 0.f;
}

void launch_copy_or_zero(float *dst, const float *src, size_t n, hipStream_t st) {
    if (dst && n) hipLaunchKernelGGL(copy_or_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                                     dst, src, n);
}

static bool dtype_ok(int dt) { return dt == DT_F32 || dt == DT_BF16 || dt == DT_F16; }

static int check_shape(int B, int T, int Hk, int Hv, int Dk, int Dv, int chunk, int gate, int form) {
    if (chunk <= 0) return fail(GDN_ERR_INVALID, "chunk must be a positive integer");
    if (B < 0 || T < 0) return fail(GDN_ERR_INVALID, "batch and timesteps must be non-negative");
    if (Hk <= 0 || Hv <= 0 || Dk <= 0 || Dv <= 0)
        return fail(GDN_ERR_INVALID, "head counts and head dims must be positive");
    if (Hv % Hk != 0) return fail(GDN_ERR_INVALID, "q/k head count must divide the value head count");
    if (gate != GATE_DECAY && gate != GATE_DECAY_VEC && gate != GATE_LOG && gate != GATE_LOG_VEC)
        return fail(GDN_ERR_INVALID, "Unsupported gating kind %d", gate);
    if (form != GDN_FORM_AUTO && form != GDN_FORM_RECURRENT && form != GDN_FORM_CHUNK)
        return fail(GDN_ERR_INVALID, "unknown form %d", form);
    if (pick_lane_width(Dk) == 0) return fail(GDN_ERR_UNSUPPORTED, "key_dim %d > 256 is not supported", Dk);
    if (Hv > 65535 || B > 65535) return fail(GDN_ERR_UNSUPPORTED, "batch and value heads must be <= 65535");
    return GDN_OK;
}

// Masked calls run the chunked form as two passes (gdn_mask.hip), whose fix-up kernels hold per-head values of one
// token in LDS: Hv <= mask_max_heads().  Per-channel gates run on the chunked form with bf16 inputs and no mask
// (gdn_chunk_vg.hip).
static bool chunk_eligible(int Hv, int Dk, int Dv, int has_mask, int gate, int in_dt) {
    if (Dk != 128 || Dv != 128) return false;
    if (gate_vec(gate)) return !has_mask && chunk_vg_supported(in_dt);
    return !has_mask || Hv <= mask_max_heads();
}

// The form a (shape, mask, gate, requested form, input dtype) resolves to, or < 0 when a requested form cannot run.
static int resolve_form(int Hv, int Dk, int Dv, int has_mask, int gate, int form, int in_dt) {
    if (form == GDN_FORM_RECURRENT) return GDN_FORM_RECURRENT;
    const bool ok = chunk_eligible(Hv, Dk, Dv, has_mask, gate, in_dt);
    if (form == GDN_FORM_CHUNK) {
        if (ok) return GDN_FORM_CHUNK;
        if (Dk != 128 || Dv != 128) return fail(GDN_ERR_UNSUPPORTED, "the chunked form needs Dk = Dv = 128");
        if (gate_vec(gate))
            return fail(GDN_ERR_UNSUPPORTED, "the chunked form takes per-channel gates with bf16 inputs and no mask");
        return fail(GDN_ERR_UNSUPPORTED, "masked calls of the chunked form take Hv <= %d", mask_max_heads());
    }
    return ok ? GDN_FORM_CHUNK : GDN_FORM_RECURRENT;
}

static bool misaligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; }

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct BwdLayout {
    size_t sub, part_qk, part_gb, part_gv, total;
};

static BwdLayout bwd_layout(int B, int T, int Hv, int Dk, int Dv, int chunk, int gate) {
    const size_t nrb = (size_t)rec_bwd_row_blocks(B, Hv, Dk, Dv, gate);
    const size_t toks = (size_t)B * T * Hv;
    BwdLayout L;
    size_t off = 0;
    L.sub = off;
    off += align256(rec_sub_floats(B, Hv, Dk, Dv, T, chunk, gate) * sizeof(float));
    L.part_qk = off;
    off += align256(nrb * toks * 2 * Dk * sizeof(float));
    L.part_gb = off;
    off += align256(nrb * toks * 2 * sizeof(float));
    L.part_gv = off;
    if (gate_vec(gate)) off += align256(nrb * toks * Dk * sizeof(float));
    L.total = off;
    return L;
}

static size_t rec_saved_bytes(int B, int T, int Hv, int Dk, int Dv, int chunk) {
    const int64_t ns = T > 0 ? (int64_t)((T + chunk - 1) / chunk) - 1 : 0;
    return (size_t)(ns > 0 ? ns : 0) * B * Hv * Dv * Dk * sizeof(float);
}

// ---- chunked form: how a call is split
//
// chunk <= 64 keeps the whole tile set from forward to backward ("saved").  chunk > 64 checkpoints: the forward keeps
// only the states at every window of W = chunk rounded up to 64 tokens (ceil(T / W) - 1 fp32 snapshots, like the
// recurrent form's boundaries), and the backward rebuilds one group of windows at a time (prep, then the forward of
// every window of the group side by side from its snapshot) before running the backward stages over that group.
// A forward-only call (no saved buffer) runs group by group as well.  Groups live in the caller's workspace: the
// largest whole number of units (windows, or 64-token chunks when forward-only) that fits, capped at about
// kGroupChunkHeads chunk-heads.

constexpr int kGroupChunkHeads = 2048;

static int ck_window(int chunk) { return chunk <= kChunkC ? 0 : (chunk + kChunkC - 1) / kChunkC * kChunkC; }

static size_t ck_state_bytes(int B, int Hv) { return (size_t)B * Hv * kChunkD * kChunkD * sizeof(float); }

static size_t ck_snap_bytes(int B, int T, int Hv, int W) {
    const int nwin = (T + W - 1) / W;
    return nwin > 1 ? (size_t)(nwin - 1) * ck_state_bytes(B, Hv) : 0;
}

struct CkShape {
    int B, T, Hk, Hv;
    bool bf16;
    int vg;  // vg_kind of the gate: 0 one decay per head, 1 per-channel log decays, 2 per-channel decays
};

// Forward group workspace: the forward tile set of Tg tokens, plus two carried states between groups when no
// snapshots carry them.
static size_t ck_fwd_group_bytes(const CkShape &s, int Tg, bool ckpt) {
    return chunk_sizes(s.B, Tg, s.Hk, s.Hv, s.bf16, false, s.vg).saved + (ckpt ? 0 : 2 * align256(ck_state_bytes(s.B, s.Hv)));
}

// Backward group workspace: two carried state adjoints, the whole tile set and the backward buffers of Tg tokens.
static size_t ck_bwd_group_bytes(const CkShape &s, int Tg) {
    const ChunkSizes cs = chunk_sizes(s.B, Tg, s.Hk, s.Hv, s.bf16, true, s.vg);
    return 2 * align256(ck_state_bytes(s.B, s.Hv)) + align256(cs.saved) + cs.work;
}

// Units of u tokens per group: the target count, or fewer when the workspace is smaller; 0 when one unit does not fit.
template <class Bytes>
static int ck_group_units(const CkShape &s, int u, size_t avail, Bytes bytes) {
    const int total = (s.T + u - 1) / u;
    const size_t per_unit = (size_t)s.B * s.Hv * (u / kChunkC);
    int g = (int)std::max<size_t>(1, kGroupChunkHeads / per_unit);
    g = std::min(g, total);
    for (; g >= 1; --g)
        if (bytes(std::min(g * u, s.T)) <= avail) return g;
    return 0;
}

static size_t ck_fwd_target_bytes(const CkShape &s, int W, bool ckpt) {
    const int u = ckpt ? W : kChunkC;
    const int g = ck_group_units(s, u, SIZE_MAX, [](int) { return (size_t)0; });
    return ck_fwd_group_bytes(s, std::min(g * u, s.T), ckpt);
}

static size_t ck_bwd_target_bytes(const CkShape &s, int W) {
    const int g = ck_group_units(s, W, SIZE_MAX, [](int) { return (size_t)0; });
    return ck_bwd_group_bytes(s, std::min(g * W, s.T));
}

// ---- masked calls on the chunked form: two chunked passes over the effective gates (gdn_mask.hip)
//
// saved (training): pass 1's saved buffer (tiles or snapshots), pass 2's tiles (chunk <= 64 only: checkpointing
// rebuilds pass 2 from pass 1's snapshots, the state sequences being the same), the effective gates g', beta', and
// z and y' (fp32 [B][T][Hv][Dv], read at masked tokens).
struct MaskSaved {
    size_t p1, p2, g2, b2, Z, Yp, total;
};
static MaskSaved mask_saved(const CkShape &s, int chunk) {
    const int W = ck_window(chunk);
    const size_t tiles = chunk_sizes(s.B, s.T, s.Hk, s.Hv, s.bf16, true, s.vg).saved;
    const size_t ng = (size_t)s.B * s.T * s.Hv * 4, nv = ng * kChunkD;
    MaskSaved m{};
    size_t off = 0;
    m.p1 = off; off += align256(W ? ck_snap_bytes(s.B, s.T, s.Hv, W) : tiles);
    m.p2 = off; off += align256(W ? 0 : tiles);
    m.g2 = off; off += align256(ng);
    m.b2 = off; off += align256(ng);
    m.Z = off; off += align256(nv);
    m.Yp = off; off += align256(nv);
    m.total = off;
    return m;
}

// Backward workspace: one pass's workspace (used by both passes in turn), the passes' cotangents and their fp32
// gradients.
struct MaskWork {
    size_t pass, pass_bytes, dy1, dz, g1[6], g2[6], total;  // g1 / g2: dq, dk, dv, dg, dbeta, dS0
};
static MaskWork mask_work(const CkShape &s, int chunk) {
    const int W = ck_window(chunk);
    MaskWork m{};
    m.pass_bytes = W ? ck_bwd_target_bytes(s, W) : chunk_sizes(s.B, s.T, s.Hk, s.Hv, s.bf16, true, s.vg).work;
    const size_t nqk = (size_t)s.B * s.T * s.Hk * kChunkD * 4, ng = (size_t)s.B * s.T * s.Hv * 4, nv = ng * kChunkD;
    const size_t nst = ck_state_bytes(s.B, s.Hv);
    const size_t sizes[6] = {nqk, nqk, nv, ng, ng, nst};
    size_t off = 0;
    m.pass = off; off += align256(m.pass_bytes);
    m.dy1 = off; off += align256(nv);
    m.dz = off; off += align256(nv);
    for (int i = 0; i < 6; ++i) { m.g1[i] = off; off += align256(sizes[i]); }
    for (int i = 0; i < 6; ++i) { m.g2[i] = off; off += align256(sizes[i]); }
    m.total = off;
    return m;
}

// Forward-only workspace: g', beta', z, then the group workspace.
static size_t mask_fwd_only_head(const CkShape &s) {
    const size_t ng = (size_t)s.B * s.T * s.Hv * 4;
    return 2 * align256(ng) + align256(ng * kChunkD);
}

static size_t dt_size(int dt) { return dt == DT_F32 ? 4 : 2; }

// Gate values per (token, value head): one, or one per key channel.
static size_t gate_width(int gate) { return gate_vec(gate) ? kChunkD : 1; }

template <class P>
static P *tok_offset(P *p, size_t elems, int dt) {
    if (!p) return p;
    using C = typename std::conditional<std::is_const<P>::value, const char, char>::type;
    return reinterpret_cast<P *>(reinterpret_cast<C *>(p) + elems * dt_size(dt));
}

}  // namespace gdn

using namespace gdn;

extern "C" {

int gdn_version(void) { return (3 << 16) | 0; }

int gdn_profile_enable(int on) {
    g_prof_on.store(on != 0, std::memory_order_relaxed);
    return GDN_OK;
}

int gdn_profile_collect(int max_entries, char *names, int name_len, double *total_ms, int *counts) {
    std::vector<ProfRec> recs;
    {
        std::lock_guard<std::mutex> lk(g_prof_mu);
        recs.swap(g_prof);
    }
    std::map<std::string, std::pair<double, int>> agg;
    int rc = GDN_OK;
    for (auto &r : recs) {
        float ms = 0.f;
        if (hipEventSynchronize(r.stop) == hipSuccess && hipEventElapsedTime(&ms, r.start, r.stop) == hipSuccess) {
            auto &e = agg[r.name];
            e.first += ms;
            e.second += 1;
        } else {
            rc = fail(GDN_ERR_LAUNCH, "profiling event failed");
        }
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    if (rc) return rc;
    int n = 0;
    for (auto &kv : agg) {
        if (n >= max_entries) break;
        snprintf(names + (size_t)n * name_len, name_len, "%s", kv.first.c_str());
        total_ms[n] = kv.second.first;
        counts[n] = kv.second.second;
        ++n;
    }
    return n;
}

const char *gdn_last_error(void) { return g_err; }

int64_t gdn_num_snapshots(int T, int chunk) {
    if (chunk <= 0 || T <= 0) return 0;
    return (int64_t)((T + chunk - 1) / chunk) - 1;
}

int gdn_select_form(int Hv, int Dk, int Dv, int has_mask, int gate_kind, int form, int in_dtype) {
    g_err[0] = 0;
    if (gate_kind != GATE_DECAY && gate_kind != GATE_DECAY_VEC && gate_kind != GATE_LOG && gate_kind != GATE_LOG_VEC)
        return fail(GDN_ERR_INVALID, "Unsupported gating kind %d", gate_kind);
    if (form != GDN_FORM_AUTO && form != GDN_FORM_RECURRENT && form != GDN_FORM_CHUNK)
        return fail(GDN_ERR_INVALID, "unknown form %d", form);
    return resolve_form(Hv, Dk, Dv, has_mask, gate_kind, form, in_dtype);
}

size_t gdn_saved_bytes(int B, int T, int Hk, int Hv, int Dk, int Dv, int chunk, int gate_kind, int has_mask,
                       int form, int in_dtype) {
    if (check_shape(B, T, Hk, Hv, Dk, Dv, chunk, gate_kind, form)) return 0;
    const int f = resolve_form(Hv, Dk, Dv, has_mask, gate_kind, form, in_dtype);
    if (f < 0 || B == 0 || T == 0) return 0;
    if (f == GDN_FORM_CHUNK) {
        const int W = ck_window(chunk);
        if (has_mask) return mask_saved({B, T, Hk, Hv, in_dtype == DT_BF16, false}, chunk).total;
        if (W) return ck_snap_bytes(B, T, Hv, W);
        return chunk_sizes(B, T, Hk, Hv, in_dtype == DT_BF16, true, vg_kind(gate_kind)).saved;
    }
    return rec_saved_bytes(B, T, Hv, Dk, Dv, chunk);
}

size_t gdn_fwd_workspace_bytes(int B, int T, int Hk, int Hv, int Dk, int Dv, int chunk, int gate_kind, int has_mask,
                               int form, int in_dtype, int with_saved) {
    if (check_shape(B, T, Hk, Hv, Dk, Dv, chunk, gate_kind, form)) return 0;
    const int f = resolve_form(Hv, Dk, Dv, has_mask, gate_kind, form, in_dtype);
    if (f != GDN_FORM_CHUNK || B == 0 || T == 0) return 0;
    const int W = ck_window(chunk);
    const CkShape shp{B, T, Hk, Hv, in_dtype == DT_BF16, vg_kind(gate_kind)};
    if (has_mask) {
        // pass 2 runs forward-only when checkpointing; a forward-only call also holds g', beta' and z
        if (with_saved) return W ? std::max(ck_fwd_target_bytes(shp, W, true), ck_fwd_target_bytes(shp, W, false)) : 0;
        return mask_fwd_only_head(shp) + ck_fwd_target_bytes(shp, W, false);
    }
    if (with_saved && !W) return 0;
    return ck_fwd_target_bytes(shp, W, with_saved != 0);
}

}  // extern "C"

namespace gdn {

// Chunked forward (resolved form GDN_FORM_CHUNK, arguments checked).
static int ck_forward(const ChunkCall &base, int chunk, void *saved, size_t saved_bytes, void *ws, size_t ws_bytes,
                      hipStream_t st) {
    const int B = base.B, T = base.T, Hk = base.Hk, Hv = base.Hv;
    const CkShape shp{B, T, Hk, Hv, base.in_dt == DT_BF16, vg_kind(base.gate)};
    const int W = ck_window(chunk);
    int rc;
    if (saved && !W) {  // the whole tile set, kept for the backward
        const size_t need = chunk_sizes(B, T, Hk, Hv, shp.bf16, true, shp.vg).saved;
        if (saved_bytes < need)
            return fail(GDN_ERR_WORKSPACE, "saved buffer of %zu bytes is smaller than the %zu bytes required",
                        saved_bytes, need);
        ChunkCall cc = base;
        cc.tiles = saved;
        cc.Ts = T;
        {
            Timed tm("ck_prep", st);
            launch_chunk_stage(cc, "prep", st);
        }
        if ((rc = check_launch(st, "gdn_fwd(ck_prep)"))) return rc;
        {
            Timed tm("ck_fwd", st);
            launch_chunk_stage(cc, "fwd", st);
        }
        return check_launch(st, "gdn_fwd(ck_fwd)");
    }
    const bool ckpt = saved != nullptr;
    float *snap = static_cast<float *>(saved);
    if (ckpt && saved_bytes < ck_snap_bytes(B, T, Hv, W))
        return fail(GDN_ERR_WORKSPACE, "saved buffer of %zu bytes is smaller than the %zu bytes of snapshots",
                    saved_bytes, ck_snap_bytes(B, T, Hv, W));
    const int u = ckpt ? W : kChunkC;
    const int units = ck_group_units(shp, u, ws ? ws_bytes : 0,
                                     [&](int Tg) { return ck_fwd_group_bytes(shp, Tg, ckpt); });
    if (units == 0)
        return fail(GDN_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes of one %d-token group",
                    ws ? ws_bytes : 0, ck_fwd_group_bytes(shp, std::min(u, T), ckpt), u);
    const int Gt = units * u;
    const size_t sb = align256(ck_state_bytes(B, Hv)), S = (size_t)B * Hv * kChunkD * kChunkD;
    char *w8 = static_cast<char *>(ws);
    float *carry[2] = {nullptr, nullptr};
    if (!ckpt) {
        carry[0] = reinterpret_cast<float *>(w8);
        carry[1] = reinterpret_cast<float *>(w8 + sb);
        w8 += 2 * sb;
    }
    for (int g = 0, ts = 0; ts < T; ++g, ts += Gt) {
        const int Tg = std::min(Gt, T - ts);
        const bool last = ts + Tg >= T;
        ChunkCall cc = base;
        cc.q = tok_offset(base.q, (size_t)ts * Hk * kChunkD, base.in_dt);
        cc.k = tok_offset(base.k, (size_t)ts * Hk * kChunkD, base.in_dt);
        cc.v = tok_offset(base.v, (size_t)ts * Hv * kChunkD, base.in_dt);
        cc.g = base.g + (size_t)ts * Hv * gate_width(base.gate);
        cc.beta = base.beta + (size_t)ts * Hv;
        cc.y = tok_offset(base.y, (size_t)ts * Hv * kChunkD, base.out_dt);
        cc.T = Tg;
        cc.Ts = T;
        cc.tiles = w8;
        cc.fwd_only = 1;
        if (ckpt) {
            const int win0 = ts / W;
            cc.snap = snap;
            cc.wc = W / kChunkC;
            cc.win0 = win0;
            cc.state0 = g == 0 ? base.state0 : snap + (size_t)(win0 - 1) * S;
            cc.state_T = last ? base.state_T : snap + (size_t)(win0 + Gt / W - 1) * S;
        } else {
            cc.state0 = g == 0 ? base.state0 : carry[g & 1];
            cc.state_T = last ? base.state_T : carry[(g + 1) & 1];
        }
        {
            Timed tm("ck_prep", st);
            launch_chunk_stage(cc, "prep", st);
        }
        if ((rc = check_launch(st, "gdn_fwd(ck_prep)"))) return rc;
        {
            Timed tm("ck_fwd", st);
            launch_chunk_stage(cc, "fwd", st);
        }
        if ((rc = check_launch(st, "gdn_fwd(ck_fwd)"))) return rc;
    }
    return GDN_OK;
}

// Chunked backward (resolved form GDN_FORM_CHUNK, arguments checked).
static int ck_backward(const ChunkCall &base, int chunk, const void *saved, size_t saved_bytes, void *ws,
                       size_t ws_bytes, hipStream_t st) {
    const int B = base.B, T = base.T, Hk = base.Hk, Hv = base.Hv;
    const CkShape shp{B, T, Hk, Hv, base.in_dt == DT_BF16, vg_kind(base.gate)};
    const int W = ck_window(chunk);
    int rc;
    if (!W) {
        const ChunkSizes cs = chunk_sizes(B, T, Hk, Hv, shp.bf16, true, shp.vg);
        if (!saved || saved_bytes < cs.saved)
            return fail(GDN_ERR_INVALID, "the saved buffer written by gdn_fwd (%zu bytes) is required", cs.saved);
        if (!ws || ws_bytes < cs.work)
            return fail(GDN_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required", ws_bytes,
                        cs.work);
        ChunkCall cc = base;
        cc.tiles = const_cast<void *>(saved);
        cc.work = ws;
        cc.Ts = T;
        {
            Timed tm("ck_bwd_seq", st);
            launch_chunk_stage(cc, "seq", st);
        }
        if ((rc = check_launch(st, "gdn_bwd(ck_bwd_seq)"))) return rc;
        {
            Timed tm("ck_bwd_local", st);
            launch_chunk_stage(cc, "local", st);
        }
        if ((rc = check_launch(st, "gdn_bwd(ck_bwd_local)"))) return rc;
        if (shp.vg == 2) {
            Timed tm("ck_vg_dg", st);
            launch_chunk_stage(cc, "dg", st);
        }
        return check_launch(st, "gdn_bwd(ck_vg_dg)");
    }
    const size_t need_snap = ck_snap_bytes(B, T, Hv, W);
    if (need_snap && (!saved || saved_bytes < need_snap))
        return fail(GDN_ERR_INVALID, "the snapshots written by gdn_fwd (%zu bytes) are required", need_snap);
    const int units = ck_group_units(shp, W, ws ? ws_bytes : 0, [&](int Tg) { return ck_bwd_group_bytes(shp, Tg); });
    if (units == 0)
        return fail(GDN_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes of one %d-token group",
                    ws ? ws_bytes : 0, ck_bwd_group_bytes(shp, std::min(W, T)), W);
    const int Gt = units * W, ng = (T + Gt - 1) / Gt;
    const size_t sb = align256(ck_state_bytes(B, Hv));
    char *w8 = static_cast<char *>(ws);
    float *carry[2] = {reinterpret_cast<float *>(w8), reinterpret_cast<float *>(w8 + sb)};
    const ChunkSizes full = chunk_sizes(B, std::min(Gt, T), Hk, Hv, shp.bf16, true, shp.vg);
    char *tiles = w8 + 2 * sb, *work = tiles + align256(full.saved);
    for (int g = ng - 1; g >= 0; --g) {
        const int ts = g * Gt, Tg = std::min(Gt, T - ts);
        const size_t qk = (size_t)ts * Hk * kChunkD, vv = (size_t)ts * Hv * kChunkD;
        ChunkCall cc = base;
        cc.q = tok_offset(base.q, qk, base.in_dt);
        cc.k = tok_offset(base.k, qk, base.in_dt);
        cc.v = tok_offset(base.v, vv, base.in_dt);
        cc.g = base.g + (size_t)ts * Hv * gate_width(base.gate);
        cc.beta = base.beta + (size_t)ts * Hv;
        cc.dy = tok_offset(base.dy, vv, base.dy_dt);
        cc.dq = tok_offset(base.dq, qk, base.grad_dt);
        cc.dk = tok_offset(base.dk, qk, base.grad_dt);
        cc.dv = tok_offset(base.dv, vv, base.grad_dt);
        cc.dg = base.dg + (size_t)ts * Hv * gate_width(base.gate);
        cc.dbeta = base.dbeta + (size_t)ts * Hv;
        cc.T = Tg;
        cc.Ts = T;
        cc.tiles = tiles;
        cc.work = work;
        {
            Timed tm("ck_prep", st);
            launch_chunk_stage(cc, "prep", st);
        }
        if ((rc = check_launch(st, "gdn_bwd(ck_prep)"))) return rc;
        {
            ChunkCall rf = cc;  // every window of the group from its entry state: H and Delta only
            rf.recompute = 1;
            rf.snap = static_cast<float *>(const_cast<void *>(saved));
            rf.wc = W / kChunkC;
            rf.win0 = ts / W;
            rf.state0 = base.state0;
            rf.y = nullptr;
            rf.state_T = nullptr;
            Timed tm("ck_fwd_recompute", st);
            launch_chunk_stage(rf, "fwd", st);
        }
        if ((rc = check_launch(st, "gdn_bwd(ck_fwd recompute)"))) return rc;
        cc.dstate_T = g == ng - 1 ? base.dstate_T : carry[(g + 1) & 1];
        cc.dstate0 = g == 0 ? base.dstate0 : carry[g & 1];
        {
            Timed tm("ck_bwd_seq", st);
            launch_chunk_stage(cc, "seq", st);
        }
        if ((rc = check_launch(st, "gdn_bwd(ck_bwd_seq)"))) return rc;
        {
            Timed tm("ck_bwd_local", st);
            launch_chunk_stage(cc, "local", st);
        }
        if ((rc = check_launch(st, "gdn_bwd(ck_bwd_local)"))) return rc;
        if (shp.vg == 2) {
            Timed tm("ck_vg_dg", st);
            launch_chunk_stage(cc, "dg", st);
            if ((rc = check_launch(st, "gdn_bwd(ck_vg_dg)"))) return rc;
        }
    }
    return GDN_OK;
}

static char *at_off(void *base, size_t off) { return static_cast<char *>(base) + off; }

// Masked chunked forward (resolved form GDN_FORM_CHUNK, arguments checked).  base holds the caller's q, k, v, g,
// beta, state0, y, state_T and shapes.
static int ck_masked_forward(const ChunkCall &base, const uint8_t *mask, int chunk, void *saved, size_t saved_bytes,
                             void *ws, size_t ws_bytes, hipStream_t st) {
    const CkShape shp{base.B, base.T, base.Hk, base.Hv, base.in_dt == DT_BF16, vg_kind(base.gate)};
    const int W = ck_window(chunk);
    const size_t tokens = (size_t)base.B * base.T;
    float *g2, *b2, *Z, *Yp = nullptr;
    void *p1 = nullptr, *p2 = nullptr;
    size_t p1_bytes = 0, p2_bytes = 0;
    void *gws = ws;
    size_t gws_bytes = ws ? ws_bytes : 0;
    if (saved) {
        const MaskSaved m = mask_saved(shp, chunk);
        if (saved_bytes < m.total)
            return fail(GDN_ERR_WORKSPACE, "saved buffer of %zu bytes is smaller than the %zu bytes required",
                        saved_bytes, m.total);
        p1 = at_off(saved, m.p1);
        p1_bytes = m.p2 - m.p1;
        if (!W) {
            p2 = at_off(saved, m.p2);
            p2_bytes = m.g2 - m.p2;
        }
        g2 = reinterpret_cast<float *>(at_off(saved, m.g2));
        b2 = reinterpret_cast<float *>(at_off(saved, m.b2));
        Z = reinterpret_cast<float *>(at_off(saved, m.Z));
        Yp = reinterpret_cast<float *>(at_off(saved, m.Yp));
    } else {
        const size_t head = mask_fwd_only_head(shp);
        if (!ws || ws_bytes < head)
            return fail(GDN_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes a masked call needs",
                        ws ? ws_bytes : 0, head);
        const size_t ng = align256(tokens * base.Hv * 4);
        g2 = reinterpret_cast<float *>(ws);
        b2 = reinterpret_cast<float *>(at_off(ws, ng));
        Z = reinterpret_cast<float *>(at_off(ws, 2 * ng));
        gws = at_off(ws, head);
        gws_bytes = ws_bytes - head;
    }
    launch_mask_gates(base.g, base.beta, mask, g2, b2, tokens, base.Hv, base.gate, st);
    int rc = check_launch(st, "gdn_fwd(mask gates)");
    if (rc) return rc;
    // pass 2: k as the query, z = S' k (fp32); its tiles kept only without checkpointing
    ChunkCall c2 = base;
    c2.q = base.k;
    c2.g = g2;
    c2.beta = b2;
    c2.y = Z;
    c2.out_dt = DT_F32;
    c2.state_T = nullptr;
    if ((rc = ck_forward(c2, chunk, p2, p2_bytes, gws, gws_bytes, st))) return rc;
    // pass 1: y' into y, or in fp32 into Yp when the backward needs it (the fix-up then writes every y)
    ChunkCall c1 = base;
    c1.g = g2;
    c1.beta = b2;
    if (Yp) {
        c1.y = Yp;
        c1.out_dt = DT_F32;
    }
    if ((rc = ck_forward(c1, chunk, p1, p1_bytes, gws, gws_bytes, st))) return rc;
    MaskArgs ma{};
    ma.q = base.q; ma.k = base.k; ma.v = base.v; ma.g = base.g; ma.beta = base.beta; ma.mask = mask;
    ma.y = base.y; ma.Z = Z; ma.Yp = Yp;
    ma.Hk = base.Hk; ma.Hv = base.Hv; ma.Dk = kChunkD; ma.Dv = kChunkD;
    ma.in_dt = base.in_dt; ma.out_dt = base.out_dt; ma.gate = base.gate;
    {
        Timed tm("mask_fix_fwd", st);
        launch_mask_fix_fwd(ma, tokens, st);
    }
    return check_launch(st, "gdn_fwd(mask fix-up)");
}

// Masked chunked backward (resolved form GDN_FORM_CHUNK, arguments checked).
static int ck_masked_backward(const ChunkCall &base, const uint8_t *mask, int chunk, const void *saved,
                              size_t saved_bytes, void *ws, size_t ws_bytes, hipStream_t st) {
    const CkShape shp{base.B, base.T, base.Hk, base.Hv, base.in_dt == DT_BF16, vg_kind(base.gate)};
    const int W = ck_window(chunk);
    const size_t tokens = (size_t)base.B * base.T;
    const MaskSaved m = mask_saved(shp, chunk);
    if (!saved || saved_bytes < m.total)
        return fail(GDN_ERR_INVALID, "the saved buffer written by gdn_fwd (%zu bytes) is required", m.total);
    const MaskWork k = mask_work(shp, chunk);
    if (!ws || ws_bytes < k.total)
        return fail(GDN_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required", ws_bytes,
                    k.total);
    void *sv = const_cast<void *>(saved);
    const float *g2 = reinterpret_cast<const float *>(at_off(sv, m.g2));
    const float *b2 = reinterpret_cast<const float *>(at_off(sv, m.b2));
    float *wf[2][6];
    for (int i = 0; i < 6; ++i) {
        wf[0][i] = reinterpret_cast<float *>(at_off(ws, k.g1[i]));
        wf[1][i] = reinterpret_cast<float *>(at_off(ws, k.g2[i]));
    }
    MaskArgs ma{};
    ma.q = base.q; ma.k = base.k; ma.v = base.v; ma.dy = base.dy; ma.g = base.g; ma.beta = base.beta;
    ma.mask = mask;
    ma.Z = reinterpret_cast<const float *>(at_off(sv, m.Z));
    ma.Yp = reinterpret_cast<float *>(at_off(sv, m.Yp));
    ma.dy1 = reinterpret_cast<float *>(at_off(ws, k.dy1));
    ma.dz = reinterpret_cast<float *>(at_off(ws, k.dz));
    ma.Hk = base.Hk; ma.Hv = base.Hv; ma.Dk = kChunkD; ma.Dv = kChunkD;
    ma.in_dt = base.in_dt; ma.dy_dt = base.dy_dt; ma.grad_dt = base.grad_dt; ma.gate = base.gate;
    {
        Timed tm("mask_bwd_cot", st);
        launch_mask_bwd_cot(ma, tokens, st);
    }
    int rc = check_launch(st, "gdn_bwd(mask cotangents)");
    if (rc) return rc;
    const bool want_ds0 = base.dstate0 != nullptr;
    for (int pass = 0; pass < 2; ++pass) {
        ChunkCall c = base;
        c.g = g2;
        c.beta = b2;
        c.dy = pass ? ma.dz : ma.dy1;
        c.dy_dt = DT_F32;
        c.grad_dt = DT_F32;
        c.dq = wf[pass][0]; c.dk = wf[pass][1]; c.dv = wf[pass][2]; c.dg = wf[pass][3]; c.dbeta = wf[pass][4];
        c.dstate0 = want_ds0 ? wf[pass][5] : nullptr;
        if (pass) {
            c.q = base.k;           // pass 2 ran with k as its query
            c.dstate_T = nullptr;   // the final state is pass 1's
        }
        const void *ps = pass && !W ? at_off(sv, m.p2) : at_off(sv, m.p1);
        const size_t ps_bytes = pass && !W ? m.g2 - m.p2 : m.p2 - m.p1;
        if ((rc = ck_backward(c, chunk, ps, ps_bytes, at_off(ws, k.pass), k.pass_bytes, st))) return rc;
    }
    ma.dq1 = wf[0][0]; ma.dk1 = wf[0][1]; ma.dv1 = wf[0][2]; ma.dg1 = wf[0][3]; ma.dbeta1 = wf[0][4];
    ma.dq2 = wf[1][0]; ma.dk2 = wf[1][1]; ma.dv2 = wf[1][2]; ma.dg2 = wf[1][3]; ma.dbeta2 = wf[1][4];
    ma.dq = base.dq; ma.dk = base.dk; ma.dv = base.dv; ma.dg = base.dg; ma.dbeta = base.dbeta;
    {
        Timed tm("mask_bwd_combine", st);
        launch_mask_bwd_combine(ma, tokens, st);
        if (want_ds0) launch_add2(base.dstate0, wf[0][5], wf[1][5], ck_state_bytes(base.B, base.Hv) / 4, st);
    }
    return check_launch(st, "gdn_bwd(mask combine)");
}

// Fixed device scratch of gdn_fwd_noalloc: a file-scope device array, one copy per GPU, held until the process
// ends.  Host code never passes the array's name to a kernel (that is a host-side stand-in); it uses the address
// hipGetSymbolAddress returns for the current device.
constexpr size_t kNoAllocScratchBytes = 64u << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxDevices];  // device ordinal -> that device's copy of `scratch` (NULL: not looked up)

// The current device's scratch address, looked up once per device with that device current; NULL (with the
// error set) on failure.
static void *device_scratch() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
        fail(GDN_ERR_LAUNCH, "gdn_fwd_noalloc: no current HIP device");
        return nullptr;
    }
    if (dev >= kMaxDevices) {
        fail(GDN_ERR_UNSUPPORTED, "gdn_fwd_noalloc: device ordinal %d >= %d", dev, kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev]) return g_scratch_ptr[dev];
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
        fail(GDN_ERR_LAUNCH, "gdn_fwd_noalloc: hipGetSymbolAddress of the scratch failed: %s", hipGetErrorString(e));
        return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
    return ptr;
}

}  // namespace gdn

extern "C" {

int gdn_fwd_noalloc(const void *q, const void *k, const void *v, const float *g, const float *beta,
                    const float *state0, const uint8_t *mask, void *y, float *state_T, int B, int T, int Hk, int Hv,
                    int Dk, int Dv, int in_dtype, int out_dtype, int gate_kind, int form, void *stream) {
    g_err[0] = 0;
    int rc = check_shape(B, T, Hk, Hv, Dk, Dv, kChunkC, gate_kind, form);
    if (rc) return rc;
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(GDN_ERR_INVALID, "unknown dtype code");
    // masked calls keep the recurrent form here: the chunked form's masked passes need buffers that grow with T
    if (mask && form == GDN_FORM_CHUNK)
        return fail(GDN_ERR_UNSUPPORTED, "gdn_fwd_noalloc runs masked calls in the recurrent form only");
    if (mask) form = GDN_FORM_RECURRENT;
    const int f = resolve_form(Hv, Dk, Dv, mask != nullptr, gate_kind, form, in_dtype);
    if (f < 0) return f;
    void *ws = nullptr;
    size_t ws_bytes = 0;
    if (f == GDN_FORM_CHUNK && B > 0 && T > 0) {
        const CkShape shp{B, T, Hk, Hv, in_dtype == DT_BF16, vg_kind(gate_kind)};
        const size_t one = ck_fwd_group_bytes(shp, std::min(kChunkC, T), false);
        if (one > kNoAllocScratchBytes)
            return fail(GDN_ERR_UNSUPPORTED,
                        "gdn_fwd_noalloc: one 64-token group of %d x %d heads needs %zu bytes; the fixed scratch "
                        "holds %zu (use gdn_fwd with a workspace)", B, Hv, one, kNoAllocScratchBytes);
        ws = device_scratch();
        if (!ws) return GDN_ERR_LAUNCH;
        ws_bytes = kNoAllocScratchBytes;
    }
    // the forward-only call of gdn_fwd, with the fixed scratch as its workspace
    return gdn_fwd(q, k, v, g, beta, state0, mask, y, state_T, nullptr, 0, ws, ws_bytes, B, T, Hk, Hv, Dk, Dv,
                   kChunkC, in_dtype, out_dtype, gate_kind, form, stream);
}

int gdn_fwd(const void *q, const void *k, const void *v, const float *g, const float *beta,
            const float *state0, const uint8_t *mask, void *y, float *state_T, void *saved, size_t saved_bytes,
            void *workspace, size_t workspace_bytes, int B, int T, int Hk, int Hv, int Dk, int Dv, int chunk,
            int in_dtype, int out_dtype, int gate_kind, int form, void *stream) {
    g_err[0] = 0;
    int rc = check_shape(B, T, Hk, Hv, Dk, Dv, chunk, gate_kind, form);
    if (rc) return rc;
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(GDN_ERR_INVALID, "unknown dtype code");
    const int f = resolve_form(Hv, Dk, Dv, mask != nullptr, gate_kind, form, in_dtype);
    if (f < 0) return f;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (B == 0) return GDN_OK;
    if (T == 0) {
        launch_copy_or_zero(state_T, state0, (size_t)B * Hv * Dv * Dk, st);
        return check_launch(st, "gdn_fwd(T=0)");
    }
    if (!q || !k || !v || !g || !beta || !y) return fail(GDN_ERR_INVALID, "null input or output pointer");
    if (f == GDN_FORM_CHUNK) {
        if (misaligned16(q) || misaligned16(k) || misaligned16(v))
            return fail(GDN_ERR_INVALID, "the chunked form needs 16-byte aligned q, k and v");
        ChunkCall cc{};
        cc.q = q; cc.k = k; cc.v = v; cc.g = g; cc.beta = beta; cc.state0 = state0;
        cc.y = y; cc.state_T = state_T;
        cc.B = B; cc.T = T; cc.Ts = T; cc.Hk = Hk; cc.Hv = Hv; cc.in_dt = in_dtype; cc.out_dt = out_dtype;
        cc.gate = gate_kind;
        if (mask) return ck_masked_forward(cc, mask, chunk, saved, saved_bytes, workspace, workspace_bytes, st);
        return ck_forward(cc, chunk, saved, saved_bytes, workspace, workspace_bytes, st);
    }
    const size_t need = rec_saved_bytes(B, T, Hv, Dk, Dv, chunk);
    float *snaps = nullptr;
    if (saved) {
        if (saved_bytes < need)
            return fail(GDN_ERR_WORKSPACE, "saved buffer of %zu bytes is smaller than the %zu bytes required",
                        saved_bytes, need);
        snaps = static_cast<float *>(saved);
    }
    RecFwdArgs a{q, k, v, g, beta, state0, mask, y, state_T, snaps,
                 B, T, Hk, Hv, Dk, Dv, chunk, in_dtype, out_dtype, gate_kind};
    {
        Timed tm("rec_fwd", st);
        launch_rec_fwd(a, st);
    }
    return check_launch(st, "gdn_fwd");
}

int gdn_decode_step(const void *q, const void *k, const void *v, const float *g, const float *beta,
                    const float *state_in, float *state_out, void *y, int B, int Hk, int Hv, int Dk, int Dv,
                    int in_dtype, int out_dtype, int gate_kind, void *stream) {
    g_err[0] = 0;
    int rc = check_shape(B, 1, Hk, Hv, Dk, Dv, 1, gate_kind, GDN_FORM_RECURRENT);
    if (rc) return rc;
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(GDN_ERR_INVALID, "unknown dtype code");
    if (B == 0) return GDN_OK;
    if (!q || !k || !v || !g || !beta || !y || !state_out)
        return fail(GDN_ERR_INVALID, "null input or output pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    // one token of the recurrent form: every thread reads its state elements before writing the same ones, so
    // state_out may be state_in
    RecFwdArgs a{q, k, v, g, beta, state_in, nullptr, y, state_out, nullptr,
                 B, 1, Hk, Hv, Dk, Dv, 1, in_dtype, out_dtype, gate_kind};
    {
        Timed tm("rec_decode", st);
        launch_rec_decode(a, st);
    }
    return check_launch(st, "gdn_decode_step");
}

size_t gdn_bwd_workspace_bytes(int B, int T, int Hk, int Hv, int Dk, int Dv, int chunk, int gate_kind,
                               int has_mask, int form, int in_dtype) {
    if (check_shape(B, T, Hk, Hv, Dk, Dv, chunk, gate_kind, form)) return 0;
    const int f = resolve_form(Hv, Dk, Dv, has_mask, gate_kind, form, in_dtype);
    if (f < 0) return 0;
    if (f == GDN_FORM_CHUNK) {
        if (B == 0 || T == 0) return 0;
        const int W = ck_window(chunk);
        if (has_mask) return mask_work({B, T, Hk, Hv, in_dtype == DT_BF16, false}, chunk).total;
        if (W) return ck_bwd_target_bytes({B, T, Hk, Hv, in_dtype == DT_BF16, vg_kind(gate_kind)}, W);
        return chunk_sizes(B, T, Hk, Hv, in_dtype == DT_BF16, true, vg_kind(gate_kind)).work;
    }
    return bwd_layout(B, T, Hv, Dk, Dv, chunk, gate_kind).total;
}

int gdn_bwd(const void *q, const void *k, const void *v, const float *g, const float *beta,
            const float *state0, const uint8_t *mask, const void *saved, size_t saved_bytes, const void *dy,
            const float *dstate_T, void *dq, void *dk, void *dv, float *dg, float *dbeta, float *dstate0,
            void *workspace, size_t workspace_bytes, int B, int T, int Hk, int Hv, int Dk, int Dv, int chunk,
            int in_dtype, int dy_dtype, int grad_dtype, int gate_kind, int form, void *stream) {
    g_err[0] = 0;
    int rc = check_shape(B, T, Hk, Hv, Dk, Dv, chunk, gate_kind, form);
    if (rc) return rc;
    if (!dtype_ok(in_dtype) || !dtype_ok(dy_dtype) || !dtype_ok(grad_dtype))
        return fail(GDN_ERR_INVALID, "unknown dtype code");
    const int f = resolve_form(Hv, Dk, Dv, mask != nullptr, gate_kind, form, in_dtype);
    if (f < 0) return f;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (B == 0) return GDN_OK;
    if (T == 0) {
        launch_copy_or_zero(dstate0, dstate_T, (size_t)B * Hv * Dv * Dk, st);
        return check_launch(st, "gdn_bwd(T=0)");
    }
    if (!q || !k || !v || !g || !beta || !dy || !dq || !dk || !dv || !dg || !dbeta)
        return fail(GDN_ERR_INVALID, "null input or output pointer");
    if (f == GDN_FORM_CHUNK) {
        if (in_dtype == DT_BF16 && dy_dtype == DT_F16)
            return fail(GDN_ERR_UNSUPPORTED, "the chunked form with bf16 inputs takes a bf16 or fp32 dy, not fp16");
        if (misaligned16(q) || misaligned16(k) || misaligned16(v) || misaligned16(dy))
            return fail(GDN_ERR_INVALID, "the chunked form needs 16-byte aligned q, k, v and dy");
        if (misaligned16(dq) || misaligned16(dk) || misaligned16(dv))
            return fail(GDN_ERR_INVALID, "the chunked form needs 16-byte aligned dq, dk and dv");
        ChunkCall cc{};
        cc.q = q; cc.k = k; cc.v = v; cc.g = g; cc.beta = beta; cc.state0 = state0;
        cc.dy = dy; cc.dstate_T = dstate_T; cc.dq = dq; cc.dk = dk; cc.dv = dv; cc.dg = dg; cc.dbeta = dbeta;
        cc.dstate0 = dstate0;
        cc.B = B; cc.T = T; cc.Ts = T; cc.Hk = Hk; cc.Hv = Hv; cc.in_dt = in_dtype; cc.dy_dt = dy_dtype;
        cc.grad_dt = grad_dtype; cc.gate = gate_kind;
        if (mask) return ck_masked_backward(cc, mask, chunk, saved, saved_bytes, workspace, workspace_bytes, st);
        return ck_backward(cc, chunk, saved, saved_bytes, workspace, workspace_bytes, st);
    }
    const size_t need_saved = rec_saved_bytes(B, T, Hv, Dk, Dv, chunk);
    if (need_saved && (!saved || saved_bytes < need_saved))
        return fail(GDN_ERR_INVALID, "the saved buffer written by gdn_fwd (%zu bytes) is required", need_saved);
    const size_t need_ws = bwd_layout(B, T, Hv, Dk, Dv, chunk, gate_kind).total;
    if (workspace_bytes < need_ws || (need_ws && !workspace))
        return fail(GDN_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required",
                    workspace_bytes, need_ws);
    RecBwdArgs a{};
    a.q = q; a.k = k; a.v = v; a.g = g; a.beta = beta; a.state0 = state0; a.mask = mask;
    a.snaps = static_cast<const float *>(saved); a.dy = dy; a.dstate_T = dstate_T;
    a.dq = dq; a.dk = dk; a.dv = dv; a.dg = dg; a.dbeta = dbeta; a.dstate0 = dstate0;
    a.B = B; a.T = T; a.Hk = Hk; a.Hv = Hv; a.Dk = Dk; a.Dv = Dv; a.chunk = chunk;
    a.in_dt = in_dtype; a.dy_dt = dy_dtype; a.grad_dt = grad_dtype; a.gate = gate_kind;
    const BwdLayout L = bwd_layout(B, T, Hv, Dk, Dv, chunk, gate_kind);
    char *ws = static_cast<char *>(workspace);
    a.ws_sub = reinterpret_cast<float *>(ws + L.sub);
    a.part_qk = reinterpret_cast<float *>(ws + L.part_qk);
    a.part_gb = reinterpret_cast<float *>(ws + L.part_gb);
    a.part_gv = reinterpret_cast<float *>(ws + L.part_gv);
    a.nrb = rec_bwd_row_blocks(B, Hv, Dk, Dv, gate_kind);
    a.max_sub = rec_max_sub(T, chunk);
    {
        Timed tm("rec_bwd", st);
        launch_rec_bwd(a, st);
    }
    rc = check_launch(st, "gdn_bwd");
    if (rc) return rc;
    {
        Timed tm("rec_bwd_reduce", st);
        launch_rec_bwd_reduce(a, st);
    }
    return check_launch(st, "gdn_bwd_reduce");
}

// ------------------------------------------------------------------------------------------- block ops

static bool all_aligned16(std::initializer_list<const void *> ps) {
    for (const void *p : ps)
        if (p && misaligned16(p)) return false;
    return true;
}

static size_t floats_bytes(size_t n) { return align256(n * sizeof(float)); }

int gdn_gates_fwd(const void *a, const void *b, const float *A_log, const float *dt_bias, float *g, float *beta,
                  int64_t tokens, int Hv, int in_dtype, int log_space, int allow_neg_eigval, void *stream) {
    g_err[0] = 0;
    if (tokens < 0 || Hv <= 0) return fail(GDN_ERR_INVALID, "tokens must be >= 0 and Hv > 0");
    if (Hv > gates_max_heads()) return fail(GDN_ERR_UNSUPPORTED, "Hv > %d is not supported", gates_max_heads());
    if (!dtype_ok(in_dtype)) return fail(GDN_ERR_INVALID, "unknown dtype code");
    if (tokens == 0) return GDN_OK;
    if (!a || !b || !A_log || !dt_bias || !g || !beta) return fail(GDN_ERR_INVALID, "null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    {
        Timed tm("gates_fwd", st);
        launch_gates_fwd(a, b, A_log, dt_bias, g, beta, (size_t)tokens, Hv, in_dtype, log_space != 0,
                         allow_neg_eigval ? 2.f : 1.f, st);
    }
    return check_launch(st, "gdn_gates_fwd");
}

size_t gdn_gates_bwd_workspace_bytes(int64_t tokens, int Hv) {
    if (tokens < 0 || Hv <= 0) return 0;
    return floats_bytes(gates_bwd_work_floats((size_t)tokens, Hv));
}

int gdn_gates_bwd(const void *a, const void *b, const float *A_log, const float *dt_bias, const float *g,
                  const float *dg, const float *dbeta, void *da, void *db, float *dA_log, float *ddt_bias,
                  void *workspace, size_t workspace_bytes, int64_t tokens, int Hv, int in_dtype, int grad_dtype,
                  int log_space, int allow_neg_eigval, void *stream) {
    g_err[0] = 0;
    if (tokens < 0 || Hv <= 0) return fail(GDN_ERR_INVALID, "tokens must be >= 0 and Hv > 0");
    if (Hv > gates_max_heads()) return fail(GDN_ERR_UNSUPPORTED, "Hv > %d is not supported", gates_max_heads());
    if (!dtype_ok(in_dtype) || !dtype_ok(grad_dtype)) return fail(GDN_ERR_INVALID, "unknown dtype code");
    if (!A_log || !dt_bias || !dA_log || !ddt_bias) return fail(GDN_ERR_INVALID, "null pointer");
    if (tokens > 0 && (!a || !b || !g || !dg || !dbeta || !da || !db)) return fail(GDN_ERR_INVALID, "null pointer");
    const size_t need = gdn_gates_bwd_workspace_bytes(tokens, Hv);
    if (need && (!workspace || workspace_bytes < need))
        return fail(GDN_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required",
                    workspace_bytes, need);
    hipStream_t st = static_cast<hipStream_t>(stream);
    {
        Timed tm("gates_bwd", st);
        launch_gates_bwd(a, b, A_log, dt_bias, g, dg, dbeta, da, db, dA_log, ddt_bias, static_cast<float *>(workspace),
                         (size_t)tokens, Hv, in_dtype, grad_dtype, log_space != 0, allow_neg_eigval ? 2.f : 1.f, st);
    }
    return check_launch(st, "gdn_gates_bwd");
}

int gdn_l2norm_fwd(const void *x, void *y, int64_t rows, int D, float eps, float scale, int dtype, void *stream) {
    g_err[0] = 0;
    if (rows < 0 || D <= 0) return fail(GDN_ERR_INVALID, "rows must be >= 0 and D > 0");
    if (!dtype_ok(dtype)) return fail(GDN_ERR_INVALID, "unknown dtype code");
    if (rows == 0) return GDN_OK;
    if (!x || !y) return fail(GDN_ERR_INVALID, "null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    {
        Timed tm("l2norm_fwd", st);
        launch_l2norm_fwd(x, y, (size_t)rows, D, eps, scale, dtype, all_aligned16({x, y}), st);
    }
    return check_launch(st, "gdn_l2norm_fwd");
}

int gdn_l2norm_bwd(const void *x, const void *dy, void *dx, int64_t rows, int D, float eps, float scale, int dtype,
                   int dy_dtype, void *stream) {
    g_err[0] = 0;
    if (rows < 0 || D <= 0) return fail(GDN_ERR_INVALID, "rows must be >= 0 and D > 0");
    if (!dtype_ok(dtype) || !dtype_ok(dy_dtype)) return fail(GDN_ERR_INVALID, "unknown dtype code");
    if (rows == 0) return GDN_OK;
    if (!x || !dy || !dx) return fail(GDN_ERR_INVALID, "null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    {
        Timed tm("l2norm_bwd", st);
        launch_l2norm_bwd(x, dy, dx, (size_t)rows, D, eps, scale, dtype, dy_dtype, all_aligned16({x, dy, dx}), st);
    }
    return check_launch(st, "gdn_l2norm_bwd");
}

static int check_conv(int B, int T, int C, int K, int dtype) {
    if (B < 0 || T < 0 || C < 0) return fail(GDN_ERR_INVALID, "B, T and C must be >= 0");
    if (K < 2) return fail(GDN_ERR_INVALID, "the conv kernel size K must be >= 2");
    if (K > conv_kmax()) return fail(GDN_ERR_UNSUPPORTED, "conv kernel size K > %d is not supported", conv_kmax());
    if (!dtype_ok(dtype)) return fail(GDN_ERR_INVALID, "unknown dtype code");
    return GDN_OK;
}

int gdn_conv_silu_fwd(const void *x, const float *w, const float *state_in, void *out, float *state_out, int B,
                      int T, int C, int K, int dtype, void *stream) {
    g_err[0] = 0;
    int rc = check_conv(B, T, C, K, dtype);
    if (rc) return rc;
    if (B == 0 || C == 0) return GDN_OK;
    if (!w || (T > 0 && (!x || !out))) return fail(GDN_ERR_INVALID, "null pointer");
    if (state_out && state_out == state_in) return fail(GDN_ERR_INVALID, "state_out must not alias state_in");
    hipStream_t st = static_cast<hipStream_t>(stream);
    ConvCall c{};
    c.x = x; c.w = w; c.state_in = state_in; c.v = out; c.state_out = state_out;
    c.B = B; c.T = T; c.C = C; c.K = K; c.qk = 0; c.Dk = 0; c.dt = dtype; c.g_dt = dtype;
    c.vec = all_aligned16({x, out});
    {
        Timed tm("conv_fwd", st);
        launch_conv_fwd(c, st);
    }
    return check_launch(st, "gdn_conv_silu_fwd");
}

size_t gdn_conv_silu_bwd_workspace_bytes(int B, int T, int C, int K) {
    if (B < 0 || T < 0 || C < 0 || K < 2) return 0;
    return floats_bytes(conv_bwd_work_floats(B, T, C, K));
}

int gdn_conv_silu_bwd(const void *x, const float *w, const float *state_in, const void *dout, void *dx, float *dw,
                      void *workspace, size_t workspace_bytes, int B, int T, int C, int K, int dtype, int dout_dtype,
                      void *stream) {
    g_err[0] = 0;
    int rc = check_conv(B, T, C, K, dtype);
    if (rc) return rc;
    if (!dtype_ok(dout_dtype)) return fail(GDN_ERR_INVALID, "unknown dtype code");
    if (C == 0) return GDN_OK;
    if (!w || !dw || (B > 0 && T > 0 && (!x || !dout || !dx))) return fail(GDN_ERR_INVALID, "null pointer");
    const size_t need = gdn_conv_silu_bwd_workspace_bytes(B, T, C, K);
    if (need && (!workspace || workspace_bytes < need))
        return fail(GDN_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required",
                    workspace_bytes, need);
    hipStream_t st = static_cast<hipStream_t>(stream);
    ConvCall c{};
    c.x = x; c.w = w; c.state_in = state_in; c.v = const_cast<void *>(dout); c.dx = dx; c.dw = dw;
    c.work = static_cast<float *>(workspace);
    c.B = B; c.T = T; c.C = C; c.K = K; c.qk = 0; c.Dk = 0; c.dt = dtype; c.g_dt = dout_dtype;
    c.vec = all_aligned16({x, dout, dx});
    {
        Timed tm("conv_bwd", st);
        launch_conv_bwd(c, st);
    }
    return check_launch(st, "gdn_conv_silu_bwd");
}

static int check_conv_qkv(int B, int T, int Hk, int Dk, int Hv, int Dv, int K, int dtype, int g_dtype, bool vec) {
    if (Hk <= 0 || Dk <= 0 || Hv <= 0 || Dv <= 0) return fail(GDN_ERR_INVALID, "head counts and dims must be > 0");
    const int64_t C = 2LL * Hk * Dk + (int64_t)Hv * Dv;
    if (C > (1 << 30)) return fail(GDN_ERR_INVALID, "too many channels");
    int rc = check_conv(B, T, (int)C, K, dtype);
    if (rc) return rc;
    if (!dtype_ok(g_dtype)) return fail(GDN_ERR_INVALID, "unknown dtype code");
    if (!conv_qkv_supported(Dk, K, dtype, g_dtype, vec, (int)C))
        return fail(GDN_ERR_UNSUPPORTED,
                    "the fused conv + L2 norm needs K = 4, 16-byte aligned buffers, channels a multiple of 4 and "
                    "Dk / (channels per lane) a power of two in [4, 64]; use gdn_conv_silu_* and gdn_l2norm_*");
    return GDN_OK;
}

int gdn_conv_qkv_fwd(const void *x, const float *w, const float *state_in, void *q, void *k, void *v,
                     float *state_out, int B, int T, int Hk, int Dk, int Hv, int Dv, int K, float q_scale, float eps,
                     int dtype, void *stream) {
    g_err[0] = 0;
    int rc = check_conv_qkv(B, T, Hk, Dk, Hv, Dv, K, dtype, dtype, all_aligned16({x, q, k, v}));
    if (rc) return rc;
    if (B == 0) return GDN_OK;
    if (!w || (T > 0 && (!x || !q || !k || !v))) return fail(GDN_ERR_INVALID, "null pointer");
    if (state_out && state_out == state_in) return fail(GDN_ERR_INVALID, "state_out must not alias state_in");
    hipStream_t st = static_cast<hipStream_t>(stream);
    ConvCall c{};
    c.x = x; c.w = w; c.state_in = state_in; c.q = q; c.k = k; c.v = v; c.state_out = state_out;
    c.B = B; c.T = T; c.C = 2 * Hk * Dk + Hv * Dv; c.K = K; c.qk = Hk * Dk; c.Dk = Dk; c.dt = dtype; c.g_dt = dtype;
    c.scale_q = q_scale; c.eps = eps; c.vec = true;
    {
        Timed tm("conv_qkv_fwd", st);
        launch_conv_fwd(c, st);
    }
    return check_launch(st, "gdn_conv_qkv_fwd");
}

int gdn_conv_qkv_bwd(const void *x, const float *w, const float *state_in, const void *dq, const void *dk,
                     const void *dv, void *dx, float *dw, void *workspace, size_t workspace_bytes, int B, int T,
                     int Hk, int Dk, int Hv, int Dv, int K, float q_scale, float eps, int dtype, int g_dtype,
                     void *stream) {
    g_err[0] = 0;
    int rc = check_conv_qkv(B, T, Hk, Dk, Hv, Dv, K, dtype, g_dtype, all_aligned16({x, dq, dk, dv, dx}));
    if (rc) return rc;
    const int C = 2 * Hk * Dk + Hv * Dv;
    if (!w || !dw || (B > 0 && T > 0 && (!x || !dq || !dk || !dv || !dx))) return fail(GDN_ERR_INVALID, "null pointer");
    const size_t need = gdn_conv_silu_bwd_workspace_bytes(B, T, C, K);
    if (need && (!workspace || workspace_bytes < need))
        return fail(GDN_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required",
                    workspace_bytes, need);
    hipStream_t st = static_cast<hipStream_t>(stream);
    ConvCall c{};
    c.x = x; c.w = w; c.state_in = state_in;
    c.q = const_cast<void *>(dq); c.k = const_cast<void *>(dk); c.v = const_cast<void *>(dv);
    c.dx = dx; c.dw = dw; c.work = static_cast<float *>(workspace);
    c.B = B; c.T = T; c.C = C; c.K = K; c.qk = Hk * Dk; c.Dk = Dk; c.dt = dtype; c.g_dt = g_dtype;
    c.scale_q = q_scale; c.eps = eps; c.vec = true;
    {
        Timed tm("conv_qkv_bwd", st);
        launch_conv_bwd(c, st);
    }
    return check_launch(st, "gdn_conv_qkv_bwd");
}

static int check_grms(int64_t rows, int D, int dtype, int z_dtype, bool bwd) {
    if (rows < 0 || D <= 0) return fail(GDN_ERR_INVALID, "rows must be >= 0 and D > 0");
    if (bwd && D > grms_dmax())
        return fail(GDN_ERR_UNSUPPORTED, "gated RMSNorm backward of rows longer than %d", grms_dmax());
    if (!dtype_ok(dtype) || !dtype_ok(z_dtype)) return fail(GDN_ERR_INVALID, "unknown dtype code");
    return GDN_OK;
}

int gdn_gated_rmsnorm_fwd(const void *y, const void *z, const float *w, void *out, int64_t rows, int D, float eps,
                          int dtype, int z_dtype, void *stream) {
    g_err[0] = 0;
    int rc = check_grms(rows, D, dtype, z_dtype, false);
    if (rc) return rc;
    if (rows == 0) return GDN_OK;
    if (!y || !z || !w || !out) return fail(GDN_ERR_INVALID, "null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    {
        Timed tm("grms_fwd", st);
        launch_grms_fwd(y, z, w, out, (size_t)rows, D, eps, dtype, z_dtype, all_aligned16({y, z, w, out}), st);
    }
    return check_launch(st, "gdn_gated_rmsnorm_fwd");
}

size_t gdn_gated_rmsnorm_bwd_workspace_bytes(int64_t rows, int D) {
    if (rows < 0 || D <= 0) return 0;
    return floats_bytes(grms_bwd_work_floats((size_t)rows, D));
}

int gdn_gated_rmsnorm_bwd(const void *y, const void *z, const float *w, const void *dout, void *dy, void *dz,
                          float *dw, void *workspace, size_t workspace_bytes, int64_t rows, int D, float eps,
                          int dtype, int z_dtype, int dout_dtype, void *stream) {
    g_err[0] = 0;
    int rc = check_grms(rows, D, dtype, z_dtype, true);
    if (rc) return rc;
    if (!dtype_ok(dout_dtype)) return fail(GDN_ERR_INVALID, "unknown dtype code");
    if (!w || !dw || (rows > 0 && (!y || !z || !dout || !dy || !dz))) return fail(GDN_ERR_INVALID, "null pointer");
    const size_t need = gdn_gated_rmsnorm_bwd_workspace_bytes(rows, D);
    if (need && (!workspace || workspace_bytes < need))
        return fail(GDN_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu bytes required",
                    workspace_bytes, need);
    hipStream_t st = static_cast<hipStream_t>(stream);
    {
        Timed tm("grms_bwd", st);
        launch_grms_bwd(y, z, w, dout, dy, dz, dw, static_cast<float *>(workspace), (size_t)rows, D, eps, dtype,
                        z_dtype, dout_dtype, all_aligned16({y, z, w, dout, dy, dz}), st);
    }
    return check_launch(st, "gdn_gated_rmsnorm_bwd");
}

}  // extern "C"
