"""The one-launch few-row kernel (batched decode and prefills of B x T <= 16
rows, ``rows_mk.hip``) against the CPU oracle and against the multi-launch
path on the same inputs.

Bars are those of the batched multi-launch path (``test_gpu_model.py``): the
matrix stages multiply f32 activations as f16 parts plus f16 remainders, so
logits are held to 1e-2 abs + 1e-3 rel of the fp32-math oracle and the fp32
wkv state to 1e-4 relative per layer and row; the fp16
token-shift states to 2e-2 abs. The two HIP paths sum in different orders,
so they agree with each other to the same bars.
"""

from __future__ import annotations

import pytest
import torch

from oracle import rwkv7_ref as R
from rwkv_tl_amd import RWKV7HIP, State
from rwkv_tl_amd.checkpoint import make_random_state_dict
from rwkv_tl_amd.weight import RWKV7Weight

pytestmark = pytest.mark.gpu

LOGIT_ATOL, LOGIT_RTOL = 1e-2, 1e-3
STATE_REL = 1e-4

_CACHE: dict[str, tuple] = {}


def _setup(shape, cuda):
    if shape not in _CACHE:
        _CACHE.clear()
        sd = make_random_state_dict(shape, seed=0, dtype=torch.float16)
        w = RWKV7Weight.from_state_dict(sd, device=cuda, dtype=torch.float16)
        model = RWKV7HIP(w, is_torch_compile=False)
        ref = R.Weights.from_emb(sd, w.emb.cpu(), torch.float32)
        _CACHE[shape] = (w, model, ref)
    return _CACHE[shape]


def _rel(x, y):
    return float((x.double() - y.double()).norm() / y.double().norm().clamp_min(1e-30))


def _check_logits(got, ref, label):
    got, ref = got.float().cpu(), ref.float().cpu()
    assert torch.isfinite(got).all(), f"{label}: non-finite logits"
    bad = (got - ref).abs() > LOGIT_ATOL + LOGIT_RTOL * ref.abs()
    assert not bool(bad.any()), f"{label}: {int(bad.sum())} logits off, max |d|={(got - ref).abs().max():.3e}"


def _check_state(S: State, ref, B, label):
    for i in range(len(S.tmix)):
        for b in range(B):
            r = _rel(S.tmix[i]["rnn"][b].cpu(), ref[0][i]["rnn"][b])
            assert r < STATE_REL, f"{label}: layer {i} row {b} rnn rel err {r:.2e}"
        xt = (S.tmix[i]["x"].cpu().float() - ref[0][i]["x"].float()).abs().max()
        xc = (S.cmix[i]["x"].cpu().float() - ref[1][i]["x"].float()).abs().max()
        assert xt <= 2e-2 and xc <= 2e-2, f"{label}: layer {i} shift state off ({xt:.2e}, {xc:.2e})"


@pytest.mark.parametrize("shape,B,steps", [("tiny", 16, 3), ("0.4b", 16, 2), ("0.4b", 3, 2)])
def test_rows_batched_decode_matches_oracle(shape, B, steps, cuda):
    print(f"rows decode {shape} B={B} steps={steps}", flush=True)
    w, model, ref_w = _setup(shape, cuda)
    model.decode_path = "auto"
    assert model.decode_launches(B) == 1, "the few-row kernel should serve this batch"
    V = w.head.shape[0]
    g = torch.Generator().manual_seed(100 + B)
    toks = torch.randint(0, V, (steps, B), generator=g)
    S = State(w.L, w.C, 64, device=cuda, batch=B)
    ref = R.new_state(w.L, w.C, dtype=torch.float16, batch=B)
    errs0 = model.last_error()
    for step in range(steps):
        lg, S = model.decode(toks[step].to(cuda), S)
        l32, ref = R.decode(ref_w, toks[step], ref)
        for b in range(B):
            _check_logits(lg[b], l32[b], f"{shape} B={B} step {step} row {b}")
    _check_state(S, ref, B, f"{shape} B={B}")
    assert model.last_error() == errs0, "a few-row launch aborted"


@pytest.mark.parametrize("shape,B,T", [("tiny", 1, 16), ("tiny", 4, 3), ("0.4b", 1, 8), ("0.4b", 1, 16),
                                       ("0.4b", 2, 8)])
def test_rows_prefill_then_decode_matches_oracle(shape, B, T, cuda):
    print(f"rows prefill {shape} B={B} T={T}", flush=True)
    w, model, ref_w = _setup(shape, cuda)
    model.decode_path = "auto"
    V = w.head.shape[0]
    g = torch.Generator().manual_seed(7 * T + B)
    prompt = torch.randint(0, V, (B, T), generator=g)
    nxt = torch.randint(0, V, (B,), generator=g)
    S = State(w.L, w.C, 64, device=cuda, batch=B)
    errs0 = model.last_error()
    model.prefill(prompt.to(cuda), S)
    ref = R.new_state(w.L, w.C, dtype=torch.float16, batch=B)
    R.prefill(ref_w, prompt, ref)
    _check_state(S, ref, B, f"{shape} B={B} T={T} after prefill")
    lg, S = model.decode(nxt.to(cuda), S)
    l32, ref = R.decode(ref_w, nxt, ref)
    for b in range(B):
        _check_logits(lg[b], l32[b], f"{shape} B={B} T={T} next-token row {b}")
    assert model.last_error() == errs0, "a few-row launch aborted"


@pytest.mark.parametrize("B,T", [(16, 1), (1, 12), (3, 5)])
def test_rows_kernel_agrees_with_multi_launch_path(B, T, cuda):
    """The same prefill / decode on the one-launch kernel and on the
    multi-launch path (model flag): logits and states agree."""
    print(f"rows vs multi-launch B={B} T={T}", flush=True)
    w, model, _ = _setup("0.4b", cuda)
    V = w.head.shape[0]
    g = torch.Generator().manual_seed(31 * B + T)
    prompt = torch.randint(0, V, (B, T), generator=g)
    nxt = torch.randint(0, V, (B,), generator=g)
    out = {}
    for path in ("auto", "kernels"):
        model.decode_path = path
        S = State(w.L, w.C, 64, device=cuda, batch=B)
        model.prefill(prompt.to(cuda), S)
        lg, S = model.decode(nxt.to(cuda), S)
        out[path] = (lg.float().cpu(), S)
    model.decode_path = "auto"
    la, Sa = out["auto"]
    lk, Sk = out["kernels"]
    bad = (la - lk).abs() > 2 * LOGIT_ATOL + LOGIT_RTOL * lk.abs()
    assert not bool(bad.any()), f"{int(bad.sum())} logits differ, max {(la - lk).abs().max():.3e}"
    for i in range(w.L):
        for b in range(B):
            r = _rel(Sa.tmix[i]["rnn"][b].cpu(), Sk.tmix[i]["rnn"][b].cpu())
            assert r < STATE_REL, f"layer {i} row {b}: {r:.2e}"
        assert (Sa.cmix[i]["x"].float() - Sk.cmix[i]["x"].float()).abs().max() <= 2e-2


def test_rows_kernel_declines_what_it_does_not_serve(cuda):
    w, model, _ = _setup("0.4b", cuda)
    model.decode_path = "auto"
    assert model.decode_launches(16) == 1
    assert model.decode_launches(17) > 1  # more than 16 rows: multi-launch path
    model.decode_path = "kernels"
    assert model.decode_launches(16) > 1
    model.decode_path = "auto"


def _rows_sync_offset(d) -> int:
    """Byte offset of the few-row kernel's sync words in the workspace: after
    the batch-1 kernel's exchange region (sync and start words, then 8
    replicas of x, proj, core and hid as 8-byte words) and the GEMM split-K
    counters, each rounded up to 256 bytes. The test checks it against the
    epoch word before using it."""
    al = lambda x: (x + 255) // 256 * 256  # noqa: E731
    C, F = d.n_embd, d.n_ffn
    SR = d.rank_w + d.rank_a + d.rank_v + d.rank_g
    mk = 256 + 4 * 1024 + (8 * C + 8 * (3 * C + SR) + 8 * C + 8 * F) * 8
    return al(mk) + al(1024 * 4)


def test_rows_kernel_abort_is_visible(cuda):
    """The few-row kernel's abort word is set from the host for the next
    launch, so every bounded wait gives up at once and every workgroup exits
    normally: NaN logits, the State unchanged, the launch counted in the
    workspace's error word; the next step runs normally and matches the
    oracle."""
    w, model, ref_w = _setup("tiny", cuda)
    model.decode_path = "auto"
    B = 4
    if model.decode_launches(B) != 1:
        pytest.skip("the few-row kernel does not fit this device")
    V = w.head.shape[0]
    g = torch.Generator().manual_seed(44)
    toks = torch.randint(0, V, (3, B), generator=g)
    S = State(w.L, w.C, 64, device=cuda, batch=B)
    ref = R.new_state(w.L, w.C, dtype=torch.float16, batch=B)
    ws = model.workspace(B, 1)
    off = _rows_sync_offset(model.dev.dims)
    words = ws[off:off + 64].view(torch.int32)
    torch.cuda.synchronize()
    e0 = int(words[0].item())
    _, S = model.decode(toks[0].to(cuda), S)
    _, ref = R.decode(ref_w, toks[0], ref)
    torch.cuda.synchronize()
    epoch = int(words[0].item())
    assert epoch == e0 + 1, "the epoch word did not advance: wrong offset"
    errs0 = model.last_error()
    before = [a.clone() for a in S.arenas]
    words[4] = epoch + 1  # abort word (byte 16) = this launch's epoch + 1
    lg, S = model.decode(toks[1].to(cuda), S)
    torch.cuda.synchronize()
    assert bool(torch.isnan(lg.float()).all()), "aborted launch must write NaN logits"
    for a, b in zip(S.arenas, before):
        assert torch.equal(a, b), "aborted launch must leave the State unchanged"
    assert model.last_error() == errs0 + 1
    lg, S = model.decode(toks[2].to(cuda), S)
    l32, ref = R.decode(ref_w, toks[2], ref)
    for b in range(B):
        _check_logits(lg[b], l32[b], f"row {b} after an aborted launch")
    assert model.last_error() == errs0 + 1


def test_rows_prefill_abort_raises_with_check_errors(cuda):
    """A prefill writes no logits, so an aborted few-row prefill shows only in
    the workspace's error word. With ``check_errors`` the model reads it after
    the call and raises; the next prefill runs normally and raises nothing."""
    from rwkv_tl_amd._lib import HipError

    w, model, ref_w = _setup("tiny", cuda)
    model.decode_path = "auto"
    if model.decode_launches(2) != 1:
        pytest.skip("the few-row kernel does not fit this device")
    V = w.head.shape[0]
    g = torch.Generator().manual_seed(45)
    toks = torch.randint(0, V, (24,), generator=g).to(cuda)
    S = State(w.L, w.C, 64, device=cuda)
    ws = model.workspace(1, 8)
    words = ws[_rows_sync_offset(model.dev.dims):][:64].view(torch.int32)
    e0 = int(words[0].item())
    model.prefill(toks[:8], S)
    torch.cuda.synchronize()
    epoch = int(words[0].item())
    assert epoch == e0 + 1, "the epoch word did not advance: wrong offset"
    model.check_errors = True
    try:
        model.raise_if_aborted()  # nothing pending
        words[4] = epoch + 1  # abort word (byte 16) = the next launch's epoch + 1
        with pytest.raises(HipError, match="aborted"):
            model.prefill(toks[8:16], S)
        model.prefill(toks[16:24], S)
    finally:
        model.check_errors = False
