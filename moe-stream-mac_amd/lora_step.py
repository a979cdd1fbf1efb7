"""LoRA training steps on this package's torch Qwen3.5 model with the reference's env-gated GDN installs
(counterpart of tools/ft_lora_lowmem.py:22-80 and of the trainer-step memory harness tools/mem_trainer.py).

    python moe-stream-mac_amd/lora_step.py --steps 4 --tokens 512 --hidden 256 --layers 4 --lora-layers 2

GDN_CHECKPOINT (default "1") installs gdn_checkpoint, GDN_VJP (default "0") installs gdn_vjp and
FROZEN_GDN_KERNEL (default "0") marks the frozen lower GDN layers with frozen_gdn, in the reference's order.
The model is random-initialised (no checkpoint is loaded) and trained with AdamW on synthetic next-token data.
Prints the reference's timing line and peak memory (torch's HIP caching-allocator counter).
"""

from __future__ import annotations

import argparse
import os
import sys
import time

import torch
import torch.nn.functional as F

import qwen3_5 as Q


def build_model(args: argparse.Namespace, dev: torch.device) -> Q.Model:
    torch.manual_seed(args.seed)
    margs = Q.ModelArgs(hidden_size=args.hidden, intermediate_size=2 * args.hidden, num_hidden_layers=args.layers,
                        num_attention_heads=args.heads, vocab_size=args.vocab,
                        linear_num_key_heads=args.key_heads, linear_num_value_heads=args.value_heads,
                        linear_key_head_dim=args.head_dim, linear_value_head_dim=args.head_dim,
                        full_attention_interval=args.full_attention_interval)
    model = Q.Model(margs)
    Q.linear_to_lora_layers(model, args.lora_layers, rank=args.rank, scale=args.scale)
    return model.to(device=dev, dtype=torch.bfloat16 if args.bf16 else torch.float32)


def install_from_env(model: Q.Model) -> list[str]:
    done = []
    if os.environ.get("GDN_CHECKPOINT", "1") == "1":
        import gdn_checkpoint
        gdn_checkpoint.install()
        done.append("gdn_checkpoint")
    if os.environ.get("GDN_VJP", "0") == "1":
        import gdn_vjp
        gdn_vjp.install()
        done.append("gdn_vjp")
    if os.environ.get("FROZEN_GDN_KERNEL", "0") == "1":
        import frozen_gdn
        frozen_gdn.install(model)
        done.append("frozen_gdn")
    return done


def main(argv: list[str] | None = None) -> int:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--steps", type=int, default=4)
    p.add_argument("--batch", type=int, default=1)
    p.add_argument("--tokens", type=int, default=512)
    p.add_argument("--hidden", type=int, default=256)
    p.add_argument("--layers", type=int, default=4)
    p.add_argument("--heads", type=int, default=4)
    p.add_argument("--key-heads", type=int, default=2)
    p.add_argument("--value-heads", type=int, default=4)
    p.add_argument("--head-dim", type=int, default=128)
    p.add_argument("--full-attention-interval", type=int, default=4)
    p.add_argument("--vocab", type=int, default=1000)
    p.add_argument("--lora-layers", type=int, default=2)
    p.add_argument("--rank", type=int, default=16)
    p.add_argument("--scale", type=float, default=20.0)
    p.add_argument("--lr", type=float, default=1e-4)
    p.add_argument("--bf16", action="store_true")
    p.add_argument("--seed", type=int, default=0)
    args = p.parse_args(argv)
    if args.steps <= 0 or args.tokens <= 1:
        p.error("steps must be positive and tokens at least 2")
    if not torch.cuda.is_available():
        print("lora_step needs a ROCm GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    model = build_model(args, dev)
    installed = install_from_env(model)
    params = [p_ for p_ in model.parameters() if p_.requires_grad]
    opt = torch.optim.AdamW(params, lr=args.lr)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    data = torch.randint(0, args.vocab, (args.batch, args.tokens + 1), device=dev, generator=gen)
    inputs, targets = data[:, :-1], data[:, 1:]
    print(f"installed: {', '.join(installed) or 'none'}; trainable parameters "
          f"{sum(p_.numel() for p_ in params)}", flush=True)
    torch.cuda.reset_peak_memory_stats(dev)
    torch.cuda.synchronize(dev)
    started = time.perf_counter()
    for step in range(args.steps):
        loss = F.cross_entropy(model(inputs).float().flatten(0, 1), targets.flatten())
        opt.zero_grad(set_to_none=True)
        loss.backward()
        opt.step()
        print(f"step {step + 1}: loss {loss.item():.4f}", flush=True)
    torch.cuda.synchronize(dev)
    elapsed = time.perf_counter() - started
    print(f"training_seconds={elapsed:.3f} training_steps={args.steps} s_per_step={elapsed / args.steps:.3f}")
    peak = torch.cuda.max_memory_allocated(dev)
    print(f"peak_memory_bytes={peak} peak_memory_gib={peak / 1024 ** 3:.3f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
