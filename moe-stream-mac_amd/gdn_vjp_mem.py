"""Isolated GDN backward memory probe at the model's real head sizes (counterpart of tools/gdn_vjp_mem.py).

    python moe-stream-mac_amd/gdn_vjp_mem.py 4096 [--impl chunked|staged|kernel|ops]

Runs one forward + VJP of gated_delta_chunked (or, for ``ops``, the differentiable gated_delta_ops) on B=1,
Hk=16, Hv=32, D=128 bf16 q/k/v (L2-normalised, q scaled by D^-1/2), decays ~ U(0.9, 1), beta ~ U(0.05, 0.95)
and a zero fp32 state, with the loss y.sum() + S_T.sum() (tools/gdn_vjp_mem.py:23-58), and prints the peak
device memory above the inputs in the reference's format.  The reference reads MLX's peak-memory counter; this
reads torch's (HIP caching allocator).
"""

from __future__ import annotations

import argparse
import sys

import torch

import gated_delta
import gdn_vjp

BATCH, KEY_HEADS, VALUE_HEADS, HEAD_DIM = 1, 16, 32, 128


def _inputs(timesteps: int, dev: torch.device):
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    shape_k = (BATCH, timesteps, KEY_HEADS, HEAD_DIM)
    shape_v = (BATCH, timesteps, VALUE_HEADS, HEAD_DIM)
    q = torch.randn(shape_k, device=dev, generator=gen)
    k = torch.randn(shape_k, device=dev, generator=gen)
    q = (q / torch.sqrt((q * q).sum(-1, keepdim=True) + 1e-6) * HEAD_DIM ** -0.5).bfloat16()
    k = (k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6)).bfloat16()
    v = torch.randn(shape_v, device=dev, generator=gen).bfloat16()
    g = 0.9 + 0.1 * torch.rand((BATCH, timesteps, VALUE_HEADS), device=dev, generator=gen)
    beta = 0.05 + 0.9 * torch.rand((BATCH, timesteps, VALUE_HEADS), device=dev, generator=gen)
    state = torch.zeros((BATCH, VALUE_HEADS, HEAD_DIM, HEAD_DIM), device=dev, dtype=torch.float32)
    return q, k, v, g, beta, state


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("timesteps", type=int)
    parser.add_argument("--impl", choices=("ops", "chunked", "staged", "kernel"), default="chunked")
    args = parser.parse_args(argv)
    if args.timesteps <= 0:
        parser.error("timesteps must be positive")
    if not torch.cuda.is_available():
        print("gdn_vjp_mem needs a ROCm GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    q, k, v, g, beta, state = _inputs(args.timesteps, dev)
    leaves = [t.requires_grad_(True) for t in (q, k, v, g, beta)]
    torch.cuda.synchronize(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    if args.impl == "ops":
        y, final_state = gated_delta.gated_delta_ops(q, k, v, g, beta, state, None)
    else:
        y, final_state = gdn_vjp.gated_delta_chunked(q, k, v, g, beta, state, None, chunk=gdn_vjp.DEFAULT_CHUNK,
                                                     impl=args.impl)
    loss = y.float().sum() + final_state.sum()
    grads = torch.autograd.grad(loss, leaves)
    torch.cuda.synchronize(dev)
    peak = torch.cuda.max_memory_allocated(dev) - base
    del grads
    mib = peak / 2 ** 20
    print(f"T={args.timesteps} impl={args.impl}: backward_peak={mib:.0f} MiB MiB_per_token={mib / args.timesteps:.2f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
