#!/usr/bin/env python3
"""GDN forward + VJP throughput on one MI355X.

A step is one forward of the delta-rule recurrence over a batch of synthetic input plus its full VJP (dq, dk,
dv, dg, dbeta, dS0), with every input already resident in HBM.  Prints ONE JSON line.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--batch B] [--chunk N] [--no-cpu-baseline]

Workloads (one GPU; the default is the T=4096 configuration the metric is quoted on):
  bf16_b4_t4096   B=4, T=4096, Hk=16, Hv=32, D=128, bf16 q/k/v/dO, fp32 state and gates, chunk 64
  bf16_b1_t4096   B=1, T=4096, same heads, bf16 q/k/v/dO
  fp32_b1_t4096   B=1, T=4096, same heads, fp32
  fp32_b1_t2048   B=1, T=2048, fp32, S0 ~ N(0, 0.02), full dS0
  ckpt_b1_t16384  B=1, T=16384, fp32, snapshots every 256 tokens, peak HBM reported
  masked_bf16_b4_t4096
                  bf16_b4_t4096 with a mask (each sequence's last 10% masked, padding): two chunked
                  passes plus the masked tokens' fix-up
  vgate_bf16_b4_t4096
                  bf16_b4_t4096 with one log decay per key channel (g [B, T, Hv, D], the headline's gate
                  distribution per channel, taken as log decays as the headline takes its per-head gates); the
                  chunked form with the per-channel-gate prep and local kernels (GDN_FORM=recurrent: the
                  token-recurrent form)
  vgate_decay_bf16_b4_t4096
                  the same gates given as decays (exp of those log decays), the reference's convention for
                  per-channel gates: d/d(decay) adds the ck_vg_dg pass
  fwd_bf16_b4_t4096
                  the forward alone, as frozen layers and prefill run it (no autograd graph, no saved tiles),
                  bf16_b4_t4096's shape
  decode_bf16_b64 one decode step (gdn_decode_step: a token of each of 64 sequences, forward only, the fp32
                  state [64, 32, 128, 128] read and written in place); bound by the state's HBM traffic
  stream_ops_bf16_b2_t8192
                  the streaming kernels around the recurrence on block-shaped bf16 inputs (B=2, T=8192, Hk=16,
                  Hv=32, D=128): fused conv + SiLU + split + q/k L2 norm, plain conv + SiLU (8192 channels), q/k L2
                  norm, gates, gated RMSNorm; a step is each forward and its backward once
  block_bf16_b2_t8192
                  one whole GDN block (projections with LoRA rank 16, conv1d K=4 + SiLU, q/k L2 norm, gates,
                  recurrence, gated RMSNorm * SiLU(z), out-projection), B=2, T=8192, hidden 2048, bf16 weights
                  and activations; a step is forward + backward to the LoRA parameters and the input
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "moe-stream-mac_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "GDN fwd+VJP tokens/sec at T=4096 (1 GPU) + % of HBM/MFMA roofline"
PEAK_HBM_GBS = 8000.0
PEAK_FP32_TFLOPS = 157.3
PEAK_BF16_TFLOPS = 2500.0
CK_C = 64


def algo_model(w, form="chunk"):
    """Algorithmic work per token of one fwd+VJP, as the roofline accounting of the measured path states it:

    bf16 chunked form (bf16 q/k/v/dO/y/dq/dk/dv, fp32 gates and their gradients):
      bytes 2 * (4 Hk D + 4 Hv D) + 4 * 4 Hv  (= 49,664 B at Hk=16, Hv=32, D=128);
      flops per head-token: intra-chunk contractions 10 C D forward, x3 with the backward; state contractions
      6 D^2 forward, x3 with the backward.  The chunked kernels run both on bf16 MFMA (the state operands are cast to
      bf16 hi / lo pairs), so both are priced at the bf16 dense peak.
    fp32 (recurrent arithmetic): bytes 4 * (4 Hk D + 4 Hv D + 4 Hv) (= 98,816 B); flops 27 D^2 per head-token
      (7 D^2 forward + 20 D^2 backward), priced at the fp32 peak.
    The recurrent form (head sizes other than 128; per-channel gates with fp32 inputs or a mask) computes the
    recurrence itself, 27 D^2 flops per head-token on fp32 VALU, whatever the input dtype; its bytes follow the
    dtype as above.
    Per-channel (vector) gates read g and write dg per key channel: 4 * 2 Hv D bytes in place of 4 * 2 Hv.
    A forward-only call (no saved state) reads q, k, v, g, beta and writes y, with the forward's third of the
    contractions (10 C D + 6 D^2 per head-token on the chunked form).
    The per-sequence state traffic (S0, S_T, dS_T, dS0) and snapshot traffic are not algorithmic, except in a decode
    step (one token per sequence, forward only), where reading and writing the fp32 state is the work:
    4 * 2 Hv D^2 + dtype * (2 Hk D + 2 Hv D) + 4 * 2 Hv bytes and 7 D^2 Hv flops per token."""
    Hk, Hv, D, C = w["Hk"], w["Hv"], w["D"], CK_C
    if w.get("forward_only"):  # a forward with no saved state (frozen layers, prefill): reads q/k/v/g/beta, writes y
        b = 2 if w["dtype"] == "bf16" else 4
        nbytes = b * (2 * Hk * D + 2 * Hv * D) + 4 * 2 * Hv
        if form == "chunk" and w["dtype"] == "bf16":
            return nbytes, {"bf16_intra_chunk": 10 * C * D * Hv, "bf16_state": 6 * D * D * Hv}, PEAK_BF16_TFLOPS
        return nbytes, {"fp32": 7 * D * D * Hv}, PEAK_FP32_TFLOPS
    if w.get("decode"):
        b = 2 if w["dtype"] == "bf16" else 4
        return (4 * 2 * Hv * D * D + b * (2 * Hk * D + 2 * Hv * D) + 4 * 2 * Hv, {"fp32": 7 * D * D * Hv},
                PEAK_FP32_TFLOPS)
    if form == "recurrent":
        b = 2 if w["dtype"] == "bf16" else 4
        gates = 4 * 2 * Hv * (D + 1) if w.get("vector_gate") else 4 * 4 * Hv
        return b * (4 * Hk * D + 4 * Hv * D) + gates, {"fp32": 27 * D * D * Hv}, PEAK_FP32_TFLOPS
    if w["dtype"] == "bf16":
        gates = 4 * 2 * Hv * (D + 1) if w.get("vector_gate") else 4 * 4 * Hv
        nbytes = 2 * (4 * Hk * D + 4 * Hv * D) + gates
        flops = {"bf16_intra_chunk": 3 * 10 * C * D * Hv, "bf16_state": 3 * 6 * D * D * Hv}
        return nbytes, flops, PEAK_BF16_TFLOPS
    nbytes = 4 * (4 * Hk * D + 4 * Hv * D + 4 * Hv)
    return nbytes, {"fp32": 27 * D * D * Hv}, PEAK_FP32_TFLOPS


def roof(nbytes, flops, peak_tflops, seconds):
    """HBM and MFMA fractions of `nbytes` / `flops` done in `seconds`; the binding roof is the larger fraction."""
    hbm = nbytes / seconds / 1e9
    fl = flops / seconds / 1e12
    f_hbm, f_fl = hbm / PEAK_HBM_GBS, fl / peak_tflops
    if f_hbm >= f_fl:
        return {"bound": "hbm", "achieved": round(hbm, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(f_hbm, 4), "other_roof_frac": round(f_fl, 4)}
    return {"bound": "mfma", "achieved": round(fl, 3), "peak": peak_tflops, "unit": "TFLOP/s",
            "frac": round(f_fl, 4), "other_roof_frac": round(f_hbm, 4)}


def kernel_model(name, B, T, Hk, Hv, D, in_b, fwd_only=False):
    """Implementation model of one launch of a kernel: (flops, HBM bytes) from what this implementation's kernel
    reads and writes, saved tiles included (recompute and padding excluded).  Chunk kernels: per (head, 64-token
    chunk); recurrent kernels: per head-token state element.  Reported beside the roofline, never as it."""
    nc = -(-T // CK_C)
    ch = B * Hv * nc            # chunk-heads
    tokh = B * T * Hv           # head-tokens
    C = CK_C
    cd, cc, dd = C * D, C * C, D * D
    bf = in_b == 2  # the bf16 path keeps bf16 operand tiles (hi / lo where split) and bf16 states
    if name == "ck_prep":
        f = ch * 4 * 2 * cc * D
        if bf:  # reads q, k (per key head), v, g, beta; writes G, T (fp32), P and P^T (hi / lo), W, -W^T, K~^T, U
            #     (fp32) and Q^T (per key head)
            kv = Hk / Hv
            by = ch * (2 * cd * 2 * kv + cd * 2 + 2 * C * 4 + C * 8 + cc * 4 + 4 * cc * 2 + 3 * cd * 2
                       + cd * 2 * kv + cd * 4)
            # a forward-only call writes none of the backward's tiles: T, P^T, -W^T, Q^T
            return f, by - (ch * (cc * 4 + 2 * cc * 2 + cd * 2 + cd * 2 * kv) if fwd_only else 0)
        return f, ch * (3 * cd * in_b + 2 * C * 4 + 2 * cd * 4 + 2 * cc * 4 + C * 8) - (ch * cc * 4 if fwd_only else 0)
    if name in ("ck_fwd", "ck_bwd_seq"):
        f = ch * (3 * 2 * cd * D + 2 * cc * D)
        if name == "ck_fwd":
            # a forward-only call saves neither h nor Delta
            if bf:  # reads W, Q, K~^T, P (hi / lo), U, G; writes h (bf16), Delta (fp32), y
                saved = 0 if fwd_only else dd * 2 + cd * 4
                return f, ch * (3 * cd * 2 + 2 * cc * 2 + cd * 4 + C * 8 + saved + cd * 2)
            saved = 0 if fwd_only else dd * 4 + cd * 4
            return f, ch * (2 * cd * 4 + cc * 4 + 2 * cd * in_b + C * 8 + saved + cd * in_b)
        f += ch * 2 * cc * D  # TdD = T^T dDelta
        if bf:  # reads K, P^T (hi / lo), Q^T, -W^T, T^T (hi / lo), dY, G; writes dh' (bf16), TdD (fp32)
            return f, ch * (cd * 2 + 2 * cc * 2 + 2 * cd * 2 + 2 * cc * 2 + cd * 2 + C * 8 + dd * 2 + cd * 4)
        return f, ch * (2 * cc * 4 + cd * 4 + 3 * cd * in_b + C * 8 + dd * 4 + cd * 4)
    if name == "ck_bwd_local":
        # dQ, TdD h^T, dK (Dv contractions), dp, dA = TdD Delta^T, dPG K, dPG^T Q, K K^T, (M + M^T) K
        f = ch * (3 * 2 * cd * D + 6 * 2 * cc * D)
        if bf:  # reads h, dh' (bf16), Delta, TdD (fp32), P (hi / lo), G, v, dy, beta and the key head's q, k;
            #     writes dv, dg, dbeta and the key head's dq, dk (one workgroup per key head sums its value heads;
            #     the fp32 running sum between them is not counted)
            kv = Hk / Hv  # key-head rows per value head
            return f, ch * (2 * dd * 2 + 2 * cd * 4 + 2 * cc * 2 + C * 8 + 2 * cd * 2 + 2 * cd * 2 * kv
                            + C * 4 + 2 * cd * 2 * kv + cd * 2 + 2 * C * 4)
        by = ch * (2 * dd * 4 + 2 * cd * 4 + cc * 4 + C * 8 + 4 * cd * in_b + C * 4
                   + 2 * cd * 4 + cd * in_b + 2 * C * 4)
        return f, by
    if name == "ck_vg_dg":  # per-channel decays: reads RHO, SIG, G (fp32), the block sums, the 7 dP / dA blocks in
        #                    use, q and k (bf16), beta and <dh', h>; writes dg (VALU work, not counted)
        return 0, ch * (3 * cd * 4 + 8 * D * 4 + 2 * 7 * 256 * 4 + 2 * cd * 2 + C * 4 + D * 4 + cd * 4)
    if name == "rec_fwd":
        return 7 * tokh * D * D, B * T * (2 * Hk * D * in_b + Hv * D * in_b * 2 + 2 * Hv * 4)
    if name == "rec_bwd":
        return 20 * tokh * D * D, B * T * (2 * Hk * D * in_b + 3 * Hv * D * in_b + 2 * Hv * 4)
    # block ops (per launch): conv over C = 2*Hk*D + Hv*D channels; the L2 norm runs once for q and once for k
    C = 2 * Hk * D + Hv * D
    if name in ("conv_fwd", "conv_qkv_fwd"):
        return 0, B * T * C * 2 * in_b
    if name in ("conv_bwd", "conv_qkv_bwd"):
        return 0, B * T * C * 3 * in_b
    if name == "l2norm_fwd":
        return 0, B * T * Hk * D * 2 * in_b
    if name == "l2norm_bwd":
        return 0, B * T * Hk * D * 3 * in_b
    if name == "gates_fwd":
        return 0, tokh * (2 * in_b + 8)
    if name == "gates_bwd":
        return 0, tokh * (4 * in_b + 12)
    if name == "grms_fwd":
        return 0, tokh * D * 3 * in_b
    if name == "grms_bwd":
        return 0, tokh * D * 5 * in_b
    if name == "rec_decode":  # one token per sequence: the fp32 state read and written, q/k/v/y, the gates
        return 7 * tokh * D * D, B * (2 * Hv * D * D * 4 + (2 * Hk * D + 2 * Hv * D) * in_b + 2 * Hv * 4)
    return 0, 0

WORKLOADS = {
    "bf16_b4_t4096": dict(B=4, T=4096, Hk=16, Hv=32, D=128, dtype="bf16", chunk=64, s0_std=0.0),
    "bf16_b1_t4096": dict(B=1, T=4096, Hk=16, Hv=32, D=128, dtype="bf16", chunk=64, s0_std=0.0),
    "fp32_b1_t4096": dict(B=1, T=4096, Hk=16, Hv=32, D=128, dtype="fp32", chunk=64, s0_std=0.0),
    "fp32_b1_t2048": dict(B=1, T=2048, Hk=16, Hv=32, D=128, dtype="fp32", chunk=64, s0_std=0.02),
    "ckpt_b1_t16384": dict(B=1, T=16384, Hk=16, Hv=32, D=128, dtype="fp32", chunk=256, s0_std=0.0),
    "masked_bf16_b4_t4096": dict(B=4, T=4096, Hk=16, Hv=32, D=128, dtype="bf16", chunk=64, s0_std=0.0,
                                 masked_tail=0.1),
    "vgate_bf16_b4_t4096": dict(B=4, T=4096, Hk=16, Hv=32, D=128, dtype="bf16", chunk=64, s0_std=0.0,
                                vector_gate=True),
    "vgate_decay_bf16_b4_t4096": dict(B=4, T=4096, Hk=16, Hv=32, D=128, dtype="bf16", chunk=64, s0_std=0.0,
                                      vector_gate=True, decay_gate=True),
    "fwd_bf16_b4_t4096": dict(B=4, T=4096, Hk=16, Hv=32, D=128, dtype="bf16", chunk=64, s0_std=0.0,
                              forward_only=True),
    "decode_bf16_b64": dict(B=64, T=1, Hk=16, Hv=32, D=128, dtype="bf16", chunk=64, s0_std=0.02, decode=True),
    "stream_ops_bf16_b2_t8192": dict(B=2, T=8192, Hk=16, Hv=32, D=128, dtype="bf16", chunk=64, s0_std=0.0,
                                     ops=True),
    "block_bf16_b2_t8192": dict(B=2, T=8192, Hk=16, Hv=32, D=128, dtype="bf16", chunk=64, s0_std=0.0,
                                block=dict(hidden=2048, K=4, rank=16, lora_scale=20.0)),
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def make_inputs(w, dev, seed=0):
    """Synthetic inputs with the measured distributions, generated on the device (seeded)."""
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    B, T, Hk, Hv, D = w["B"], w["T"], w["Hk"], w["Hv"], w["D"]
    dt = torch.bfloat16 if w["dtype"] == "bf16" else torch.float32
    n = lambda *s: torch.randn(*s, device=dev, generator=gen)
    q, k = n(B, T, Hk, D), n(B, T, Hk, D)
    q = q * (D ** -0.5) * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6)
    k = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    v = n(B, T, Hv, D)
    beta = torch.sigmoid(n(B, T, Hv))
    A_log = torch.empty(Hv, device=dev).uniform_(0.0, float(torch.log(torch.tensor(16.0))), generator=gen)
    if w.get("vector_gate"):
        # one log decay per key channel, [B, T, Hv, D], from the same distribution; decay_gate: given as decays
        # (the reference's convention for per-channel gates, tools/gdn_vjp.py:174-179)
        g = -torch.exp(A_log)[:, None] * torch.nn.functional.softplus(n(B, T, Hv, D))
        if w.get("decay_gate"):
            g = torch.exp(g)
    else:
        g = -torch.exp(A_log) * torch.nn.functional.softplus(n(B, T, Hv))  # log decay per head
    state = n(B, Hv, D, D) * w["s0_std"] if w["s0_std"] > 0 else torch.zeros(B, Hv, D, D, device=dev)
    dy = n(B, T, Hv, D)
    return dict(q=q.to(dt), k=k.to(dt), v=v.to(dt), g=g.contiguous(), beta=beta.contiguous(),
                state=state.contiguous(), dy=dy.to(dt))


def make_block(w, dev, seed=0):
    """One GDN block with LoRA adapters on its five projections (base frozen), bf16, plus input and output
    cotangent: projection weights ~ N(0, 0.02), LoRA A ~ N(0, 0.02), B = 0; conv, A_log, dt_bias and norm weight
    at the module's initialisation."""
    import torch
    import qwen3_5 as Q
    torch.manual_seed(seed)
    bw = w["block"]
    args = Q.ModelArgs(hidden_size=bw["hidden"], linear_num_key_heads=w["Hk"], linear_num_value_heads=w["Hv"],
                       linear_key_head_dim=w["D"], linear_value_head_dim=w["D"], linear_conv_kernel_dim=bw["K"])
    blk = Q.GatedDeltaNet(args)
    with torch.no_grad():
        for m in (blk.in_proj_qkv, blk.in_proj_z, blk.in_proj_b, blk.in_proj_a, blk.out_proj):
            m.weight.normal_(0.0, 0.02)
    Q.freeze(blk)
    for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj"):
        setattr(blk, n, Q.LoRALinear(getattr(blk, n), bw["rank"], bw["lora_scale"]))
    blk = blk.to(device=dev, dtype=torch.bfloat16).train()
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    shape = (w["B"], w["T"], bw["hidden"])
    x = torch.randn(shape, device=dev, generator=gen).to(torch.bfloat16).requires_grad_(True)
    dout = torch.randn(shape, device=dev, generator=gen).to(torch.bfloat16)
    return blk, x, dout


def make_stream_ops(w, dev, seed=0):
    """Inputs, leaves and cotangents of the streaming block kernels at the workload's shape (bf16 activations,
    fp32 parameters)."""
    import torch
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    B, T, Hk, Hv, D = w["B"], w["T"], w["Hk"], w["Hv"], w["D"]
    C = 2 * Hk * D + Hv * D
    n = lambda *s: torch.randn(*s, device=dev, generator=gen)
    bf = torch.bfloat16
    x = dict(qkv=n(B, T, C).to(bf), conv_w=n(C, 4) * 0.3, qr=n(B, T, Hk, D).to(bf), kr=n(B, T, Hk, D).to(bf),
             a=n(B, T, Hv).to(bf), b=n(B, T, Hv).to(bf), A_log=torch.rand(Hv, device=dev, generator=gen) * 2.7,
             dt_bias=n(Hv) * 0.1, y=n(B, T, Hv, D).to(bf), z=n(B, T, Hv, D).to(bf), norm_w=1 + 0.1 * n(D))
    leaves = [t.requires_grad_(True) for t in x.values()]
    return x, leaves


def cpu_info():
    info = {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)), "machine": platform.machine()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                info["model"] = line.split(":", 1)[1].strip()
    except Exception:
        pass
    for var in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS"):
        if os.environ.get(var):
            info[var] = os.environ[var]
    return info


def _oracle_group_run(args):
    """One key-head group of the CPU baseline: the oracle's fwd+VJP on its value heads (worker process)."""
    T, hk, rep = args
    from oracle import gdn_oracle as O
    d = O.make_inputs(1, T, 16, 32, 128, seed=0)
    sl = slice(hk * rep, (hk + 1) * rep)
    O.gated_delta_chunked_vjp(d["q"][:, :, hk:hk + 1], d["k"][:, :, hk:hk + 1], d["v"][:, :, sl],
                              d["decay"][:, :, sl], d["beta"][:, :, sl], d["state"][:, sl], None,
                              d["dy"][:, :, sl], None, chunk=64)


def cpu_baseline(T_sample=1024, T_parallel=4096, workers=None):
    """The NumPy oracle (restating tools/gdn_vjp.py _forward + _backward, impl="staged"), fp32, chunk 64,
    B=1, Hk=16, Hv=32, D=128, on bounded samples:
      single core: the whole head set over T_sample tokens, median of 3 after one warm-up;
      all cores: the 16 key-head groups (2 value heads each) in worker processes over T_parallel tokens, the wall
      time of the slowest, median of 3 after one warm-up.
    Runs before the GPU is touched (the workers are forked)."""
    import multiprocessing as mp
    import numpy as np
    from oracle import gdn_oracle as O
    d = O.make_inputs(1, T_sample, 16, 32, 128, seed=0)
    run = lambda: O.gated_delta_chunked_vjp(d["q"], d["k"], d["v"], d["decay"], d["beta"], d["state"], None,
                                            d["dy"], None, chunk=64)
    run()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med1 = float(np.median(times))
    n = workers or min(16, len(os.sched_getaffinity(0)))
    jobs = [(T_parallel, hk, 2) for hk in range(16)]
    ptimes = []
    with mp.get_context("fork").Pool(n) as pool:
        pool.map(_oracle_group_run, [(64, hk, 2) for hk in range(16)])
        for _ in range(3):
            t0 = time.perf_counter()
            pool.map(_oracle_group_run, jobs, chunksize=1)
            ptimes.append(time.perf_counter() - t0)
    medp = float(np.median(ptimes))
    info = cpu_info()
    return {"value": round(T_parallel / medp, 1), "unit": "tokens/s", "cores": n, "kind": "port",
            "sample": f"numpy oracle fwd+VJP, B=1 T={T_parallel} Hk=16 Hv=32 D=128 fp32 chunk 64: the 16 key-head "
                      f"groups over {n} worker processes, median of 3 ({medp:.2f} s) after 1 warm-up",
            "single_core": {"value": round(T_sample / med1, 1), "unit": "tokens/s", "cores": 1,
                            "sample": f"the whole head set in one process, B=1 T={T_sample}, median of 3 "
                                      f"({med1:.2f} s) after 1 warm-up; elementwise numpy is single-threaded"},
            "host": info}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="bf16_b4_t4096", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample", type=int, default=1024)
    ap.add_argument("--batch", type=int, default=0, help="override the workload's batch size B")
    ap.add_argument("--chunk", type=int, default=0,
                    help="override the workload's chunk (the snapshot interval of the recurrent form and of the "
                         "checkpointed chunked form)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="run one plain device copy of MIB MiB first (scales rocprof FETCH/WRITE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported (the GDN path here is "
              "single-GPU; across GPUs it would shard by (batch, key-head group), which needs no exchange)",
              file=sys.stderr)
        sys.exit(2)

    cb = None
    if not args.no_cpu_baseline:
        log("bench: cpu baseline (before the GPU is initialised)")
        cb = cpu_baseline(args.cpu_sample)
        log(f"bench: cpu baseline {cb['value']} tokens/s on {cb['cores']} cores, "
            f"{cb['single_core']['value']} on one")

    import torch
    import gdn_engine
    import gdn_lib

    w = dict(WORKLOADS[args.workload])
    if args.chunk:
        w["chunk"] = args.chunk
    if args.batch:
        w["B"] = args.batch
    dev = torch.device("cuda:0")
    gdn_lib.load()
    if args.copy_calibration:
        n = args.copy_calibration * 2 ** 20 // 4
        src = torch.ones(n, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"bench: calibration copy of {args.copy_calibration} MiB done")
        del src, dst
    log(f"bench: workload {args.workload} {w}")
    B, T, Hk, Hv, D = w["B"], w["T"], w["Hk"], w["Hv"], w["D"]
    if "block" in w:
        blk, xb, dout = make_block(w, dev)
        leaves = [xb] + [p for p in blk.parameters() if p.requires_grad]

        def step():
            return torch.autograd.grad(blk(xb), leaves, dout)
    elif "ops" in w:
        import gdn_block as GB
        so, leaves = make_stream_ops(w, dev)
        cot = None

        def outputs():
            q, k, v = GB.conv_qkv(so["qkv"], so["conv_w"], Hk, D, Hv, D, D ** -0.5)
            c = GB.conv_silu(so["qkv"], so["conv_w"])
            qn, kn = GB.normalize_qk(so["qr"], so["kr"], D ** -0.5)
            g, beta = GB.gates(so["a"], so["b"], so["A_log"], so["dt_bias"])
            o = GB.gated_rmsnorm(so["y"], so["z"], so["norm_w"])
            return [q, k, v, c, qn, kn, g, beta, o]

        with torch.no_grad():
            cot = [torch.randn_like(t) for t in outputs()]

        def step():
            return torch.autograd.grad(outputs(), leaves, cot)
    elif "decode" in w:
        x = {n: t[:, 0].contiguous() if n not in ("state",) else t for n, t in make_inputs(w, dev).items()}

        def step():  # one token of each sequence, the state updated in place
            return gdn_engine.decode_step(x["q"], x["k"], x["v"], x["g"], x["beta"], x["state"], x["state"],
                                          log_gate=True, out_dtype=x["q"].dtype)
    elif "forward_only" in w:
        x = make_inputs(w, dev)

        def step():  # no autograd graph, no saved tiles: y and the final state only
            return gdn_engine.recurrence(x["q"], x["k"], x["v"], x["g"], x["beta"], x["state"], None,
                                         chunk=w["chunk"], log_gate=True, output_dtype=x["q"].dtype, need_grad=False)
    else:
        x = make_inputs(w, dev)
        out_dtype = x["q"].dtype
        leaves = [x[n].requires_grad_(True) for n in ("q", "k", "v", "g", "beta", "state")]
        mask = None
        if w.get("masked_tail"):
            mask = torch.ones(B, T, dtype=torch.bool, device=dev)
            mask[:, T - int(T * w["masked_tail"]):] = False

        log_gate = not w.get("decay_gate")

        def step():
            y, S = gdn_engine.recurrence(x["q"], x["k"], x["v"], x["g"], x["beta"], x["state"], mask,
                                         chunk=w["chunk"], log_gate=log_gate, output_dtype=out_dtype)
            return torch.autograd.grad([y], leaves, [x["dy"]])

    for i in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log("bench: warmup done")
    torch.cuda.reset_peak_memory_stats(dev)
    gdn_lib.profile_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    gdn_lib.profile_enable(False)
    kt = gdn_lib.profile_collect()
    peak_gib = torch.cuda.max_memory_allocated(dev) / 2 ** 30
    log(f"bench: timed {args.steps} steps in {elapsed:.3f} s; kernels {kt}")

    tokens = B * T
    value = tokens * args.steps / elapsed
    dom = max(kt, key=lambda n: kt[n][0])
    ms, cnt = kt[dom]
    avg_ms = ms / cnt
    in_b = 2 if w["dtype"] == "bf16" else 4
    km = lambda n: kernel_model(n, B, T, Hk, Hv, D, in_b, fwd_only=bool(w.get("forward_only")))
    step_s = elapsed / args.steps
    form = "chunk" if any(n.startswith("ck_") for n in kt) else "recurrent"
    a_bytes, a_flops, a_peak = algo_model(w, form)
    # units one launch processes: tokens of the batch per launch (a launch covers a group of tokens when the
    # call runs group-wise)
    launch_tokens = tokens * args.steps / cnt
    if "ops" in w:
        # streaming kernels: the bytes the launch must read and write, against the HBM roof
        a_bytes, a_flops = km(dom)[1] / tokens, {"none": 0}
    roofline = roof(a_bytes * launch_tokens, sum(a_flops.values()) * launch_tokens, a_peak, avg_ms * 1e-3)
    traffic = None
    tj = ROOT / "profiles" / "traffic.json"
    if tj.exists():
        rec = json.loads(tj.read_text()).get(args.workload, {}).get(dom)
        if rec:
            traffic = rec["read_bytes"] + rec["write_bytes"]
    # the implementation model of a chunk kernel covers the whole batch once; a call that runs group-wise launches
    # it several times per step, each launch over its share (a masked call's two passes each cover the whole batch)
    per_step = lambda n: kt[n][1] / args.steps / (2 if w.get("masked_tail") else 1) if n.startswith("ck_") else 1
    i_flops, i_bytes = (int(x / per_step(dom)) for x in km(dom))
    roofline.update({
        "traffic": traffic, "traffic_source": "profiles/traffic.json (rocprofv3 FETCH_SIZE + WRITE_SIZE)"
        if traffic else None, "kernel": dom, "avg_launch_ms": round(avg_ms, 4),
        "algo_bytes_per_token": a_bytes, "algo_flops_per_token": a_flops, "tokens_per_launch": launch_tokens,
        "algo_bytes_per_launch": a_bytes * launch_tokens,
        "algo_flops_per_launch": sum(a_flops.values()) * launch_tokens,
        # the whole step against the same roofline (a block step also runs the projections: no step roof there)
        "step": None if ("block" in w or "ops" in w) else dict(roof(a_bytes * tokens, sum(a_flops.values()) * tokens, a_peak,
                                                     step_s), ms=round(step_s * 1e3, 4)),
        "implementation_model": {"bytes_per_launch": i_bytes, "flops_per_launch": i_flops,
                                 "hbm_frac": round(i_bytes / (avg_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
        "kernels_ms_per_step": {n: round(v[0] / args.steps, 4) for n, v in kt.items()},
        # every kernel's modelled bytes per launch over its own average launch time
        "kernels_gbs": {n: round(km(n)[1] / per_step(n) / (v[0] / v[1] * 1e-3) / 1e9, 1)
                        for n, v in kt.items() if km(n)[1]}})
    # each kernel's own share of the step's algorithmic flops (split in proportion to the implementation model's
    # flops of the kernels) over that kernel's own time, against the same flop peak; `frac` above charges the
    # whole step's work to the dominant kernel alone
    kf = {n: km(n)[0] for n in kt}
    kf_sum = sum(kf.values())
    if kf_sum and "block" not in w and "ops" not in w:
        algo_step = sum(a_flops.values()) * tokens
        roofline["kernels_own_share_flop_frac"] = {
            n: round(algo_step * f / kf_sum / (kt[n][0] / args.steps * 1e-3) / (a_peak * 1e12), 4)
            for n, f in kf.items() if f}
    if "block" in w:
        lib_ms = sum(v[0] for v in kt.values()) / args.steps
        roofline["outside_library_ms_per_step"] = round(elapsed / args.steps * 1e3 - lib_ms, 4)
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(elapsed / args.steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16" if (w["dtype"] == "bf16" and (form == "chunk" or "ops" in w)) else "fp32",
        "data": "synthetic",
        # inputs in bf16 run in bf16 only on the chunked form: the recurrent form computes in fp32
        "config": {"workload": args.workload, "B": B, "T": T, "Hk": Hk, "Hv": Hv, "Dk": D, "Dv": D,
                   "chunk": w["chunk"], "inputs": w["dtype"], "state": "fp32", "form": form,
                   "global_batch": B, "seq_len": T, "parallelism": "single-gpu", **w.get("block", {})},
        "peak_hbm_gib": round(peak_gib, 3),
        "roofline": roofline,
    }
    if cb is not None:
        line["cpu_baseline"] = cb
        line["gpu_over_cpu"] = round(value / cb["value"], 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
