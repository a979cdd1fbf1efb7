"""Tiny-model counterparts of the reference's end-to-end tests, on this package's torch Qwen3.5 stack:

- tools/test_gdn_vjp.py:155-174 and tools/test_gdn_checkpoint.py:196-220: after install(), the loss and every
  LoRA gradient of a tiny model match those of a baseline update (GRADIENT_ATOL 1e-4).  The reference's baseline
  is mlx-lm's ops loop; here it is the independent torch statement of the recurrence in tests/naive_torch.py
  (gates from their closed form), so only the recurrence differs between the two runs.
- tools/test_frozen_gdn.py:64-97: frozen_gdn.install() on a model with a LoRA adapter in its last layer only
  sends the two lower GDN layers down the forward-only path ([True, True, False], also after model.train()),
  and loss and gradients match the un-patched model (PARITY_ATOL 1e-3).
- tools/gdn_vjp_mem.py: the memory probe's counterpart (moe-stream-mac_amd/gdn_vjp_mem.py) reports the
  backward's peak per token at the real head sizes.

The tiny model follows the reference's (tools/test_gdn_checkpoint.py:132-177): hidden 64, 4 layers, 2 key / 4
value heads of dim 8, conv kernel 4, vocabulary 1000; its MLP is dense (the MoE routing is outside the GDN path).
"""

import pytest
import torch
import torch.nn.functional as F

import naive_torch

pytestmark = pytest.mark.gpu

INPUT_IDS = [[17, 42, 81, 109, 211]]
TARGET_IDS = [[42, 81, 109, 211, 307]]
GRADIENT_ATOL = 1e-4
PARITY_ATOL = 1e-3


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    import gdn_lib
    gdn_lib.load()
    return torch.device("cuda:0")


def _naive_update(q, k, v, a, b, A_log, dt_bias, state=None, mask=None, *, use_kernel=True, lower_bound=None,
                  allow_neg_eigval=False):
    """gated_delta_update from closed-form gates and the torch recurrence of tests/naive_torch.py (fp32)."""
    beta = torch.sigmoid(b.float()) * (2.0 if allow_neg_eigval else 1.0)
    decay = torch.exp(-torch.exp(A_log.float()) * F.softplus(a.float() + dt_bias.float()))
    Bsz, _, Hv, Dv = v.shape
    if state is None:
        state = torch.zeros((Bsz, Hv, Dv, q.shape[-1]), device=q.device, dtype=torch.float32)
    return naive_torch.recurrence(q.float(), k.float(), v.float(), decay, beta, state, mask)


def _tiny_model(dev, num_lora_layers, full_attention_interval, lora_b, seed=321):
    import qwen3_5 as Q
    torch.manual_seed(seed)
    model = Q.Model(Q.ModelArgs(full_attention_interval=full_attention_interval))
    Q.linear_to_lora_layers(model, num_lora_layers)
    if lora_b == "random":  # non-zero B: the A gradients are non-zero too
        with torch.no_grad():
            for m in model.modules():
                if isinstance(m, Q.LoRALinear):
                    m.lora_b.normal_(0.0, 0.05)
    return model.to(dev)


def _loss_and_grads(model, dev):
    inputs = torch.tensor(INPUT_IDS, device=dev)
    targets = torch.tensor(TARGET_IDS, device=dev)
    params = [(n, p) for n, p in model.named_parameters() if p.requires_grad]
    loss = F.cross_entropy(model(inputs).flatten(0, 1), targets.flatten())
    grads = torch.autograd.grad(loss, [p for _, p in params])
    return loss.detach(), [(n, g.detach()) for (n, _), g in zip(params, grads)]


def _assert_close(expected, actual, atol):
    (le, ge), (la, ga) = expected, actual
    assert [n for n, _ in ge] == [n for n, _ in ga]
    diffs = [float((le - la).abs().max())] + [float((x - y).abs().max()) for (_, x), (_, y) in zip(ge, ga)]
    print(f"max abs loss / gradient difference {max(diffs):.3g} over {len(ge)} gradients", flush=True)
    torch.testing.assert_close(la, le, atol=atol, rtol=0)
    for (n, x), (_, y) in zip(ge, ga):
        torch.testing.assert_close(y, x, atol=atol, rtol=0, msg=lambda m: f"{n}: {m}")


def _patchable(monkeypatch):
    """Register every global that install() functions rebind so that the test restores them."""
    import frozen_gdn
    import gdn_checkpoint
    import gdn_vjp
    import qwen3_5 as Q
    monkeypatch.setattr(Q, "gated_delta_update", Q.gated_delta_update)
    monkeypatch.setattr(Q.GatedDeltaNet, "forward", Q.GatedDeltaNet.forward)
    for mod in (gdn_vjp, gdn_checkpoint, frozen_gdn):
        monkeypatch.setattr(mod, "_ORIGINAL_UPDATE", None)
    monkeypatch.setattr(frozen_gdn, "_ORIGINAL_GDN_CALL", None)


@pytest.mark.parametrize("lora_b", ["zero", "random"])
@pytest.mark.parametrize("which", ["gdn_vjp", "gdn_checkpoint"])
def test_install_matches_tiny_model_loss_and_lora_gradients(dev, monkeypatch, which, lora_b):
    import importlib
    import qwen3_5 as Q
    _patchable(monkeypatch)
    print(f"tiny model install {which} lora_b={lora_b}", flush=True)
    model = _tiny_model(dev, num_lora_layers=4, full_attention_interval=2, lora_b=lora_b)
    monkeypatch.setattr(Q, "gated_delta_update", _naive_update)
    expected = _loss_and_grads(model, dev)
    importlib.import_module(which).install()
    assert Q.gated_delta_update is not _naive_update
    actual = _loss_and_grads(model, dev)
    _assert_close(expected, actual, GRADIENT_ATOL)
    if lora_b == "zero":  # B = 0 gives exactly zero A gradients (tools/test_gdn_vjp.py LoRA init)
        assert all(float(g.abs().max()) == 0.0 for n, g in actual[1] if n.endswith("lora_a"))


def test_frozen_dispatch_and_parity(dev, monkeypatch):
    import frozen_gdn
    import qwen3_5 as Q
    _patchable(monkeypatch)
    print("tiny model frozen_gdn dispatch", flush=True)
    model = _tiny_model(dev, num_lora_layers=1, full_attention_interval=3, lora_b="random")
    assert [t for t in model.model.args.layer_types] == [
        "linear_attention", "linear_attention", "full_attention", "linear_attention"]
    expected = _loss_and_grads(model, dev)
    frozen_gdn.install(model)
    original = frozen_gdn._ORIGINAL_UPDATE
    assert original is not None
    calls = []

    def spy(*args, **kwargs):
        calls.append(bool(kwargs.get("use_kernel")))
        return original(*args, **kwargs)

    monkeypatch.setattr(frozen_gdn, "_ORIGINAL_UPDATE", spy)
    inputs = torch.tensor(INPUT_IDS, device=dev)
    with torch.no_grad():
        model(inputs)
    assert calls == [True, True, False]
    calls.clear()
    model.train()
    with torch.no_grad():
        model(inputs)
    assert calls == [True, True, False]
    calls.clear()
    actual = _loss_and_grads(model, dev)
    assert calls == [True, True, False]
    _assert_close(expected, actual, PARITY_ATOL)


def test_memory_probe_reports_backward_peak_per_token(dev, capsys):
    """The counterpart of tools/gdn_vjp_mem.py runs at the real head sizes and reports the backward's peak in the
    reference's format; the chunked form's saved chunk tiles and workspace stay well under 2 MiB per token (the
    reference measured 10.3 MiB per token for its kernel implementation)."""
    import re
    import gdn_vjp_mem
    print("memory probe T=1024", flush=True)
    assert gdn_vjp_mem.main(["1024"]) == 0
    out = capsys.readouterr().out
    m = re.search(r"T=1024 impl=chunked: backward_peak=(\d+) MiB MiB_per_token=([0-9.]+)", out)
    assert m, out
    assert 0.0 < float(m.group(2)) < 2.0, out


@pytest.mark.parametrize("env", [("1", "0", "0"), ("0", "1", "1")])
def test_lora_step_driver(dev, monkeypatch, capsys, env):
    """The counterpart of tools/ft_lora_lowmem.py installs what GDN_CHECKPOINT / GDN_VJP / FROZEN_GDN_KERNEL ask
    for and runs AdamW LoRA steps through the chunked form (head dim 128) with finite losses, printing the
    reference's timing line and the peak memory."""
    import math
    import re
    import lora_step
    _patchable(monkeypatch)
    names = ("GDN_CHECKPOINT", "GDN_VJP", "FROZEN_GDN_KERNEL")
    for name, value in zip(names, env):
        monkeypatch.setenv(name, value)
    print(f"lora_step env {dict(zip(names, env))}", flush=True)
    assert lora_step.main(["--steps", "2", "--tokens", "256", "--hidden", "128", "--layers", "4",
                           "--lora-layers", "2", "--bf16"]) == 0
    out = capsys.readouterr().out
    want = [m for m, v in zip(("gdn_checkpoint", "gdn_vjp", "frozen_gdn"), env) if v == "1"]
    assert f"installed: {', '.join(want)};" in out, out
    losses = [float(x) for x in re.findall(r"step \d+: loss ([0-9.]+)", out)]
    assert len(losses) == 2 and all(math.isfinite(v) for v in losses), out
    assert "training_steps=2" in out and "peak_memory_gib=" in out, out
