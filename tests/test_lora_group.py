"""The grouped LoRA projections (qwen3_5._LoRAGroupFn) against plain autograd of y = x W^T + s (x A^T) B^T, in
float64 on the CPU: outputs and the gradients of x, A, B and an unfrozen W, for groups of several projections
with different ranks and scales, a projection whose output gets no cotangent, and a single projection."""

import pytest
import torch
import torch.nn as nn

import qwen3_5 as Q


def _mods(shapes, seed):
    g = torch.Generator().manual_seed(seed)
    mods = []
    for (fan_in, fan_out, rank, scale) in shapes:
        m = Q.LoRALinear(nn.Linear(fan_in, fan_out, bias=False), rank, scale)
        with torch.no_grad():
            m.base.weight.copy_(torch.randn(fan_out, fan_in, generator=g) * 0.3)
            m.lora_a.copy_(torch.randn(rank, fan_in, generator=g) * 0.3)
            m.lora_b.copy_(torch.randn(fan_out, rank, generator=g) * 0.3)  # non-zero: every term contributes
        mods.append(m.double())
    return mods


def _plain(x, m):
    return x @ m.base.weight.t() + m.scale * (x @ m.lora_a.t()) @ m.lora_b.t()


def _grads(outs, cots, leaves):
    pairs = [(o, c) for o, c in zip(outs, cots) if c is not None]
    return torch.autograd.grad([o for o, _ in pairs], leaves, [c for _, c in pairs], allow_unused=True)


@pytest.mark.parametrize("unfreeze", [False, True])
@pytest.mark.parametrize("drop", [None, 2])
def test_group_matches_plain_autograd(unfreeze, drop):
    shapes = [(24, 40, 4, 2.0), (24, 16, 3, 0.5), (24, 5, 2, 20.0), (24, 7, 4, 1.0)]
    mods = _mods(shapes, seed=3)
    if unfreeze:
        mods[1].base.weight.requires_grad_(True)
    x = torch.randn(2, 9, 24, dtype=torch.float64, requires_grad=True)
    g = torch.Generator().manual_seed(5)
    cots = [torch.randn(2, 9, s[1], generator=g, dtype=torch.float64) for s in shapes]
    if drop is not None:
        cots[drop] = None
    leaves = [x] + [p for m in mods for p in (m.lora_a, m.lora_b)] + ([mods[1].base.weight] if unfreeze else [])
    got = Q.lora_group(x, mods)
    want = [_plain(x, m) for m in mods]
    for a, b in zip(got, want):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)
    for a, b in zip(_grads(got, cots, leaves), _grads(want, cots, leaves)):
        if b is None:
            assert a is None or torch.count_nonzero(a) == 0
        else:
            torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)


def test_single_module_and_bias_fallback():
    (m,) = _mods([(12, 6, 2, 3.0)], seed=9)
    x = torch.randn(4, 12, dtype=torch.float64, requires_grad=True)
    c = torch.randn(4, 6, dtype=torch.float64)
    got, want = m(x), _plain(x, m)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
    for a, b in zip(_grads([got], [c], [x, m.lora_a, m.lora_b]), _grads([want], [c], [x, m.lora_a, m.lora_b])):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)
    mb = Q.LoRALinear(nn.Linear(12, 6, bias=True), 2, 3.0).double()
    with torch.no_grad():
        mb.lora_b.normal_()
    ref = x @ mb.base.weight.t() + mb.base.bias + mb.scale * (x @ mb.lora_a.t()) @ mb.lora_b.t()
    torch.testing.assert_close(mb(x), ref, rtol=1e-12, atol=1e-12)
