"""CPU-side checks of the C ABI and the host logic (no kernel launches)."""

import ctypes

import pytest
import torch

import gdn_lib


def test_library_exports_every_declared_symbol():
    lib = gdn_lib.load()
    declared = gdn_lib.header_functions()
    assert {"gdn_fwd", "gdn_bwd", "gdn_bwd_workspace_bytes", "gdn_last_error", "gdn_num_snapshots",
            "gdn_version", "gdn_saved_bytes", "gdn_select_form", "gdn_profile_enable",
            "gdn_profile_collect"} <= set(declared)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.gdn_version() >> 16 == 3


def test_bindings_match_header_arities():
    """Every declared function has a ctypes binding with as many arguments as its prototype."""
    import re
    text = gdn_lib.HEADER.read_text()
    protos = re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(gdn_[a-z_0-9]+)\s*\(([^)]*)\)\s*;", text, re.M)
    assert len(protos) >= 20
    for name, params in protos:
        params = params.strip()
        n = 0 if params in ("", "void") else params.count(",") + 1
        assert name in gdn_lib._SIGS, name
        assert len(gdn_lib._SIGS[name][0]) == n, (name, len(gdn_lib._SIGS[name][0]), n)


def test_snapshot_count_matches_reference_boundaries():
    lib = gdn_lib.load()
    # the reference keeps ceil(T/chunk)+1 boundaries including S0 and S_T (tools/gdn_vjp.py:205-235)
    for T, chunk in [(1, 64), (64, 64), (65, 64), (200, 16), (4096, 64), (16384, 256), (0, 64)]:
        ref_boundaries = -(-T // chunk) + 1 if T else 1
        expect = max(ref_boundaries - 2, 0)
        assert lib.gdn_num_snapshots(T, chunk) == expect


def test_abi_rejects_bad_arguments_without_launching():
    lib = gdn_lib.load()
    null = None
    fwd = lambda *ints: lib.gdn_fwd(*([null] * 10), 0, null, 0, *ints, null)
    rc = fwd(1, 4, 2, 3, 8, 8, 0, 0, 0, 0, 0)
    assert rc == gdn_lib.GDN_ERR_INVALID
    assert b"chunk must be a positive integer" in lib.gdn_last_error()
    rc = fwd(1, 4, 2, 3, 8, 8, 64, 0, 0, 0, 0)
    assert rc == gdn_lib.GDN_ERR_INVALID and b"head count must divide" in lib.gdn_last_error()
    rc = fwd(1, 4, 1, 1, 300, 8, 64, 0, 0, 0, 0)
    assert rc == gdn_lib.GDN_ERR_UNSUPPORTED
    rc = fwd(1, 4, 1, 1, 8, 8, 64, 7, 0, 0, 0)
    assert rc == gdn_lib.GDN_ERR_INVALID and b"dtype" in lib.gdn_last_error()
    rc = fwd(1, 4, 1, 1, 8, 8, 64, 0, 0, 9, 0)
    assert rc == gdn_lib.GDN_ERR_INVALID
    rc = fwd(1, 4, 1, 1, 8, 8, 64, 0, 0, 0, 0)
    assert rc == gdn_lib.GDN_ERR_INVALID and b"null" in lib.gdn_last_error()
    # the chunked form cannot run a vector gate, and says so
    rc = fwd(1, 4, 1, 1, 128, 128, 64, 0, 0, gdn_lib.GATE_DECAY_VEC, gdn_lib.FORM_CHUNK)
    assert rc == gdn_lib.GDN_ERR_UNSUPPORTED and b"chunked form" in lib.gdn_last_error()
    # a forward-only call of the chunked form needs its group workspace; a training call its saved buffer
    fake = ctypes.c_void_p(256)   # never dereferenced: the size checks fail first
    rc = lib.gdn_fwd(*([fake] * 6), null, fake, fake, null, 0, null, 0, 1, 4, 1, 1, 128, 128, 64, 0, 0, 2, 0, null)
    assert rc == gdn_lib.GDN_ERR_WORKSPACE and b"workspace of 0 bytes" in lib.gdn_last_error()
    rc = lib.gdn_fwd(*([fake] * 6), null, fake, fake, fake, 16, null, 0, 1, 4, 1, 1, 128, 128, 64, 0, 0, 2, 0, null)
    assert rc == gdn_lib.GDN_ERR_WORKSPACE and b"saved buffer of 16 bytes" in lib.gdn_last_error()
    need = lib.gdn_bwd_workspace_bytes(1, 4, 1, 1, 8, 8, 64, 0, 0, 0, 0)
    assert need > 0 and lib.gdn_bwd_workspace_bytes(1, 4, 1, 1, 8, 8, 0, 0, 0, 0, 0) == 0
    rc = lib.gdn_bwd(*([fake] * 8), 0, *([fake] * 9), need - 1, 1, 4, 1, 1, 8, 8, 64, 0, 0, 0, 0, 0, null)
    assert rc == gdn_lib.GDN_ERR_WORKSPACE
    # per-channel decays on the chunked form need the d/d(decay) buffers beyond what log decays need
    L = gdn_lib
    ws_log = lib.gdn_bwd_workspace_bytes(2, 300, 2, 4, 128, 128, 64, L.GATE_LOG_VEC, 0, L.FORM_CHUNK, L.BF16)
    ws_dec = lib.gdn_bwd_workspace_bytes(2, 300, 2, 4, 128, 128, 64, L.GATE_DECAY_VEC, 0, L.FORM_CHUNK, L.BF16)
    assert ws_dec > ws_log > 0
    rc = lib.gdn_bwd(*([fake] * 6), null, fake, 1 << 40, fake, null, *([fake] * 6), fake, ws_log, 2, 300, 2, 4, 128,
                     128, 64, L.BF16, L.BF16, L.BF16, L.GATE_DECAY_VEC, L.FORM_CHUNK, null)
    assert rc == L.GDN_ERR_WORKSPACE and b"workspace of" in lib.gdn_last_error()
    # bf16 inputs with an fp16 cotangent cannot run on the chunked form (its kernels read bf16 or fp32 dy)
    rc = lib.gdn_bwd(*([fake] * 6), null, fake, 1 << 40, *([fake] * 9), 1 << 40, 1, 4, 1, 1, 128, 128, 64, 1, 2,
                     1, 2, gdn_lib.FORM_CHUNK, null)
    assert rc == gdn_lib.GDN_ERR_UNSUPPORTED and b"fp16" in lib.gdn_last_error()
    # B == 0 is a no-op
    assert fwd(0, 4, 1, 1, 8, 8, 64, 0, 0, 0, 0) == 0
    # the decode step checks its arguments the same way
    dec = lambda ptrs, *ints: lib.gdn_decode_step(*ptrs, *ints, null)
    assert dec([fake] * 8, 0, 1, 1, 8, 8, 0, 0, 0) == 0
    assert dec([fake] * 8, 1, 1, 1, 300, 8, 0, 0, 0) == gdn_lib.GDN_ERR_UNSUPPORTED
    assert dec([fake] * 8, 1, 2, 3, 8, 8, 0, 0, 0) == gdn_lib.GDN_ERR_INVALID
    assert dec([fake] * 7 + [null], 1, 1, 1, 8, 8, 0, 0, 0) == gdn_lib.GDN_ERR_INVALID
    assert b"null" in lib.gdn_last_error()
    assert dec([fake] * 8, 1, 1, 1, 8, 8, 0, 0, 9) == gdn_lib.GDN_ERR_INVALID


def test_noalloc_refusals_without_launching():
    """gdn_fwd_noalloc refuses, before any device call, a masked call that asks for the chunked form and a call whose
    one 64-token group does not fit its fixed scratch."""
    L = gdn_lib
    lib = L.load()
    fake = ctypes.c_void_p(256)   # never dereferenced: both calls fail their host-side checks first
    rc = lib.gdn_fwd_noalloc(*([fake] * 6), fake, fake, fake, 2, 70, 2, 4, 128, 128, L.F32, L.F32, L.GATE_LOG,
                             L.FORM_CHUNK, None)
    assert rc == L.GDN_ERR_UNSUPPORTED and b"recurrent form only" in lib.gdn_last_error()
    rc = lib.gdn_fwd_noalloc(*([fake] * 6), None, fake, fake, 16, 64, 16, 64, 128, 128, L.BF16, L.BF16, L.GATE_LOG,
                             L.FORM_CHUNK, None)
    assert rc == L.GDN_ERR_UNSUPPORTED and b"fixed scratch" in lib.gdn_last_error()


def test_block_op_abi_rejects_bad_arguments_without_launching():
    lib = gdn_lib.load()
    L = gdn_lib
    null, fake = None, ctypes.c_void_p(256)   # never dereferenced: every call below fails its checks first
    assert lib.gdn_gates_fwd(*([fake] * 6), 10, 257, 0, 0, 0, null) == L.GDN_ERR_UNSUPPORTED
    assert lib.gdn_gates_fwd(*([fake] * 6), -1, 4, 0, 0, 0, null) == L.GDN_ERR_INVALID
    assert lib.gdn_gates_fwd(*([fake] * 6), 10, 4, 5, 0, 0, null) == L.GDN_ERR_INVALID
    assert lib.gdn_gates_fwd(*([null] * 6), 10, 4, 0, 0, 0, null) == L.GDN_ERR_INVALID
    assert b"null" in lib.gdn_last_error()
    assert lib.gdn_gates_fwd(*([null] * 6), 0, 4, 0, 0, 0, null) == 0   # no tokens: nothing to do
    need = lib.gdn_gates_bwd_workspace_bytes(1000, 32)
    assert need >= 4 * 2 * 32 * 4 and need % 256 == 0
    rc = lib.gdn_gates_bwd(*([fake] * 12), need - 1, 1000, 32, 0, 0, 0, 0, null)
    assert rc == L.GDN_ERR_WORKSPACE
    assert lib.gdn_l2norm_fwd(fake, fake, 4, 0, 1e-6, 1.0, 0, null) == L.GDN_ERR_INVALID
    assert lib.gdn_l2norm_bwd(null, null, null, 4, 128, 1e-6, 1.0, 0, 0, null) == L.GDN_ERR_INVALID
    assert lib.gdn_l2norm_fwd(null, null, 0, 128, 1e-6, 1.0, 0, null) == 0
    conv = lambda B, T, C, K, dt=0, s_in=null, s_out=null: lib.gdn_conv_silu_fwd(fake, fake, s_in, fake, s_out,
                                                                                 B, T, C, K, dt, null)
    assert conv(1, 4, 8, 1) == L.GDN_ERR_INVALID and b"K must be >= 2" in lib.gdn_last_error()
    assert conv(1, 4, 8, 9) == L.GDN_ERR_UNSUPPORTED
    assert conv(1, 4, 8, 4, dt=3) == L.GDN_ERR_INVALID
    assert conv(1, 4, 8, 4, s_in=fake, s_out=fake) == L.GDN_ERR_INVALID
    assert b"alias" in lib.gdn_last_error()
    ws = lib.gdn_conv_silu_bwd_workspace_bytes(2, 8192, 8192, 4)
    assert ws == 2 * 32 * 8192 * 4 * 4   # one partial per (batch, 256 tokens) x C x K floats
    rc = lib.gdn_conv_silu_bwd(*([fake] * 7), ws - 1, 2, 8192, 8192, 4, 1, 1, null)
    assert rc == L.GDN_ERR_WORKSPACE
    assert lib.gdn_gated_rmsnorm_fwd(fake, fake, fake, fake, 4, 0, 1e-6, 0, 0, null) == L.GDN_ERR_INVALID
    rc = lib.gdn_gated_rmsnorm_bwd(*([fake] * 8), 1 << 20, 4, 4097, 1e-6, 0, 0, 0, null)
    assert rc == L.GDN_ERR_UNSUPPORTED and b"4096" in lib.gdn_last_error()
    ws = lib.gdn_gated_rmsnorm_bwd_workspace_bytes(2 * 8192 * 32, 128)
    assert ws == 2 * 8192 * 32 // 512 * 128 * 4
    rc = lib.gdn_gated_rmsnorm_bwd(*([fake] * 8), ws - 1, 2 * 8192 * 32, 128, 1e-6, 1, 1, 1, null)
    assert rc == L.GDN_ERR_WORKSPACE


def test_block_wrappers_error_on_cpu_tensors():
    import gdn_block
    x = torch.zeros(2, 4, 8)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        gdn_block.conv_silu(x, torch.zeros(8, 4))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        gdn_block.l2norm(x)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        gdn_block.gated_rmsnorm(x, x, torch.ones(8))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        gdn_block.gates(x, x, torch.zeros(8), torch.zeros(8))


def test_saved_sizes_by_form():
    lib = gdn_lib.load()
    L = gdn_lib
    rec = lib.gdn_saved_bytes(1, 4096, 16, 32, 128, 128, 64, L.GATE_LOG, 0, L.FORM_RECURRENT, L.F32)
    assert rec == 63 * 32 * 128 * 128 * 4
    ck = lib.gdn_saved_bytes(1, 4096, 16, 32, 128, 128, 64, L.GATE_LOG, 0, L.FORM_AUTO, L.F32)
    assert ck == lib.gdn_saved_bytes(1, 4096, 16, 32, 128, 128, 64, L.GATE_LOG, 0, L.FORM_CHUNK, L.F32) > rec
    assert lib.gdn_select_form(32, 128, 128, 0, L.GATE_LOG, L.FORM_AUTO, L.F32) == L.FORM_CHUNK
    assert lib.gdn_select_form(32, 128, 128, 1, L.GATE_LOG, L.FORM_AUTO, L.F32) == L.FORM_CHUNK   # masks: two chunked passes
    assert lib.gdn_select_form(32, 8, 8, 0, L.GATE_DECAY, L.FORM_AUTO, L.F32) == L.FORM_RECURRENT
    # masked calls take the chunked form up to 256 value heads; above, AUTO falls back to the recurrent form and
    # the size queries answer for that form
    assert lib.gdn_select_form(256, 128, 128, 1, L.GATE_LOG, L.FORM_AUTO, L.F32) == L.FORM_CHUNK
    assert lib.gdn_select_form(260, 128, 128, 1, L.GATE_LOG, L.FORM_AUTO, L.F32) == L.FORM_RECURRENT
    assert lib.gdn_select_form(260, 128, 128, 0, L.GATE_LOG, L.FORM_AUTO, L.F32) == L.FORM_CHUNK
    assert lib.gdn_select_form(260, 128, 128, 1, L.GATE_LOG, L.FORM_CHUNK, L.F32) == L.GDN_ERR_UNSUPPORTED
    assert b"Hv <= 256" in lib.gdn_last_error()
    # per-channel gates: the chunked form with bf16 inputs and no mask, the recurrent form otherwise
    assert lib.gdn_select_form(32, 128, 128, 0, L.GATE_DECAY_VEC, L.FORM_AUTO, L.BF16) == L.FORM_CHUNK
    assert lib.gdn_select_form(32, 128, 128, 0, L.GATE_DECAY_VEC, L.FORM_AUTO, L.F32) == L.FORM_RECURRENT
    assert lib.gdn_select_form(32, 128, 128, 1, L.GATE_DECAY_VEC, L.FORM_AUTO, L.BF16) == L.FORM_RECURRENT
    assert lib.gdn_select_form(32, 64, 64, 0, L.GATE_DECAY_VEC, L.FORM_AUTO, L.BF16) == L.FORM_RECURRENT
    assert lib.gdn_select_form(32, 128, 128, 1, L.GATE_DECAY_VEC, L.FORM_CHUNK, L.BF16) == L.GDN_ERR_UNSUPPORTED
    assert b"per-channel gates" in lib.gdn_last_error()
    # per-channel log decays resolve like per-channel decays and save the same tiles; on the chunked form the
    # backward of decays (not log decays) also keeps, per (value head, 64-token chunk), the pieces d/d(decay) is
    # formed from: two fp32 [64][128] tiles, two fp32 [4][128] block sums, dP and dA fp32 [64][64] and one fp32
    # [128] row (2 x 4 heads x 5 chunks)
    vgd = 2 * 4 * 5 * (2 * 64 * 128 + 2 * 4 * 128 + 2 * 64 * 64 + 128) * 4
    for m, dt in ((0, L.BF16), (0, L.F32), (1, L.BF16)):
        assert (lib.gdn_select_form(32, 128, 128, m, L.GATE_LOG_VEC, L.FORM_AUTO, dt)
                == lib.gdn_select_form(32, 128, 128, m, L.GATE_DECAY_VEC, L.FORM_AUTO, dt))
        saved = lambda gk: lib.gdn_saved_bytes(2, 300, 2, 4, 128, 128, 64, gk, m, L.FORM_AUTO, dt)
        assert saved(L.GATE_LOG_VEC) == saved(L.GATE_DECAY_VEC) > 0
        work = lambda gk: lib.gdn_bwd_workspace_bytes(2, 300, 2, 4, 128, 128, 64, gk, m, L.FORM_AUTO, dt)
        extra = vgd if (m, dt) == (0, L.BF16) else 0
        assert work(L.GATE_LOG_VEC) + extra == work(L.GATE_DECAY_VEC) > 0
    assert lib.gdn_select_form(32, 128, 128, 0, 4, L.FORM_AUTO, L.BF16) == L.GDN_ERR_INVALID
    for q in (lambda f: lib.gdn_saved_bytes(1, 300, 130, 260, 128, 128, 64, L.GATE_LOG, 1, f, L.BF16),
              lambda f: lib.gdn_bwd_workspace_bytes(1, 300, 130, 260, 128, 128, 64, L.GATE_LOG, 1, f, L.BF16)):
        assert q(L.FORM_AUTO) == q(L.FORM_RECURRENT) > 0
    assert lib.gdn_fwd_workspace_bytes(1, 300, 130, 260, 128, 128, 64, L.GATE_LOG, 1, L.FORM_AUTO, L.BF16, 1) == 0
    assert lib.gdn_fwd_workspace_bytes(1, 300, 130, 260, 128, 128, 64, L.GATE_LOG, 1, L.FORM_CHUNK, L.BF16, 0) == 0


def _ck_tile_bytes_per_chunk_head(bf16: bool) -> int:
    """Bytes the chunked form keeps per (head, 64-token chunk) at chunk <= 64, stated independently of the
    library: G (fp64), U, Delta (fp32 [64][128]), the entry state h, and T, plus per set
      fp32: h fp32, T, P fp32 [64][64], W fp32 [64][128];
      bf16: h bf16, T as hi / lo bf16 planes, W, (K diag(gamma_C/gamma))^T, -W^T (bf16 [64][128]), P and P^T as
            hi / lo bf16 planes, and Q^T (bf16 [128][64]) once per key head (half a tile per value head at Hv/Hk=2)."""
    C, D = 64, 128
    common = C * 8 + 2 * C * D * 4 + C * C * 4
    if bf16:
        return common + D * D * 2 + 3 * C * D * 2 + 2 * (2 * C * C * 2) + C * D * 2 // 2
    return common + D * D * 4 + C * C * 4 + C * D * 4


@pytest.mark.parametrize("dt, bf16", [(gdn_lib.F32, False), (gdn_lib.BF16, True)])
def test_chunked_saved_bytes_keep_tiles_or_snapshots(dt, bf16):
    lib = gdn_lib.load()
    L = gdn_lib
    B, T, Hk, Hv = 4, 4096, 16, 32
    full = lib.gdn_saved_bytes(B, T, Hk, Hv, 128, 128, 64, L.GATE_LOG, 0, L.FORM_CHUNK, dt)
    per = _ck_tile_bytes_per_chunk_head(bf16)
    assert full == pytest.approx(B * Hv * (T // 64) * per, rel=1e-3)
    # chunk > 64 checkpoints: ceil(T / W) - 1 fp32 states, W = chunk rounded up to a multiple of 64
    state = B * Hv * 128 * 128 * 4
    for chunk, W in [(256, 256), (100, 128), (65, 128), (4096, 4096), (5000, 5056)]:
        snaps = lib.gdn_saved_bytes(B, T, Hk, Hv, 128, 128, chunk, L.GATE_LOG, 0, L.FORM_CHUNK, dt)
        assert snaps == max(-(-T // W) - 1, 0) * state
    # chunk <= 64 always keeps the tiles
    assert lib.gdn_saved_bytes(B, T, Hk, Hv, 128, 128, 16, L.GATE_LOG, 0, L.FORM_CHUNK, dt) == full


def test_chunked_workspaces_are_bounded_by_groups():
    lib = gdn_lib.load()
    L = gdn_lib
    args = lambda T, chunk: (1, T, 16, 32, 128, 128, chunk, L.GATE_LOG, 0, L.FORM_CHUNK, L.F32)
    # full save: no forward workspace, a backward workspace that grows with T
    assert lib.gdn_fwd_workspace_bytes(*args(4096, 64), 1) == 0
    a, b = lib.gdn_bwd_workspace_bytes(*args(4096, 64)), lib.gdn_bwd_workspace_bytes(*args(8192, 64))
    assert 1.9 < b / a < 2.1
    # checkpointing and forward-only calls work group by group: the workspaces stop growing with T once a
    # group (about 2048 chunk-heads) is reached
    for fn in (lambda T: lib.gdn_bwd_workspace_bytes(*args(T, 256)),
               lambda T: lib.gdn_fwd_workspace_bytes(*args(T, 256), 1),
               lambda T: lib.gdn_fwd_workspace_bytes(*args(T, 64), 0)):
        small, big, huge = fn(1024), fn(16384), fn(65536)
        assert 0 < small < big == huge
    # the checkpointed backward workspace is well below the full-save saved buffer plus workspace at T=16384
    full = lib.gdn_saved_bytes(*args(16384, 64)) + lib.gdn_bwd_workspace_bytes(*args(16384, 64))
    ckpt = lib.gdn_saved_bytes(*args(16384, 256)) + lib.gdn_bwd_workspace_bytes(*args(16384, 256))
    assert ckpt < full / 3


def test_workspace_scales_with_row_blocks_and_tokens():
    lib = gdn_lib.load()
    a = lib.gdn_bwd_workspace_bytes(1, 4096, 16, 32, 128, 128, 64, 0, 0, 1, 0)
    b = lib.gdn_bwd_workspace_bytes(1, 8192, 16, 32, 128, 128, 64, 0, 0, 1, 0)
    assert 1.9 < b / a < 2.1


def test_python_wrapper_errors_on_cpu_tensors():
    import gdn_vjp
    q = torch.zeros(1, 4, 1, 8)
    v = torch.zeros(1, 4, 2, 8)
    g = torch.ones(1, 4, 2)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        gdn_vjp.gated_delta_chunked(q, q, v, g, g)
    with pytest.raises(ValueError, match="chunk must be a positive integer"):
        gdn_vjp.gated_delta_chunked(q, q, v, g, g, chunk=-1)
    with pytest.raises(ValueError, match="impl must be"):
        gdn_vjp.gated_delta_chunked(q, q, v, g, g, impl="nope")


def test_install_rebinds_and_delegates_use_kernel(monkeypatch):
    """tools/test_gdn_vjp.py:177-193 and tools/test_gdn_checkpoint.py:223-241, on the torch module."""
    import gdn_checkpoint
    import gdn_vjp
    import qwen3_5
    for mod, fn in ((gdn_vjp, "_vjp_update"), (gdn_checkpoint, "_checkpointed_update")):
        calls = []
        sentinel = object()

        def spy(*args, **kwargs):
            calls.append(kwargs.get("use_kernel"))
            return sentinel

        monkeypatch.setattr(mod, "_ORIGINAL_UPDATE", None)
        monkeypatch.setattr(qwen3_5, "gated_delta_update", spy)
        mod.install()
        assert qwen3_5.gated_delta_update is getattr(mod, fn)
        mod.install()   # idempotent
        assert mod._ORIGINAL_UPDATE is spy
        values = [torch.tensor(0.0) for _ in range(7)]
        assert qwen3_5.gated_delta_update(*values, use_kernel=True) is sentinel
        assert calls == [True]


def test_update_without_install_raises(monkeypatch):
    import gdn_vjp
    monkeypatch.setattr(gdn_vjp, "_ORIGINAL_UPDATE", None)
    with pytest.raises(RuntimeError, match="install\\(\\) has not been called"):
        gdn_vjp._vjp_update(*[torch.tensor(0.0)] * 7, use_kernel=True)


def test_frozen_gdn_install_errors():
    import frozen_gdn
    import qwen3_5
    with pytest.raises(TypeError, match="qwen3_5-family"):
        frozen_gdn.install(torch.nn.Linear(2, 2))
    model = qwen3_5.Model(qwen3_5.ModelArgs(full_attention_interval=3))
    qwen3_5.freeze(model)
    with pytest.raises(ValueError, match="trainable parameter"):
        frozen_gdn.install(model)
