"""The bfloat16 model (``RWKV7HIPBF16``, ``demo/rwkv7_bf16.py:18-27``) on the GPU.

Weights, shift states and logits are bfloat16; the kernels compute in fp32
and keep the wkv state in fp32, as the float16 model does. Two oracles, the
restated pure-torch model on the very same bf16 weights and embedding rows:

* ``ref32``: fp32 arithmetic, bf16 shift states. The batch-1 decode keeps
  every intermediate in fp32, so logits must agree to the rounding of a bf16
  logit (atol 1e-2 + rtol 8e-3: two half-ulps of bf16's 8-bit significand)
  and the per-layer wkv state to 1e-4 relative after the decode steps. The
  prefill and batched paths multiply f32 activations as a bf16 part plus a
  bf16 remainder (16 significant bits, measured state errors near 1e-5), so
  they are held to the same bars.
* ``refbf``: the reference's own bf16 semantics (every torch operation in
  bfloat16), compared with the reference's bf16 criterion
  (``test/test_forward.py:71-81,104-119``): max |d logit| <= 4.0, the same
  argmax and the same top-5 set -- up to near-ties: random-init logits are
  crowded (the 5th and 6th largest often differ by less than the bf16
  reference's own rounding, a few bf16 ulps), so an index may take another's
  place only where their reference logits are within tie(x) = 2e-2 + 2^-5 |x|
  (four ulps of bf16 at x, plus a floor).
"""

from __future__ import annotations

import pytest
import torch

from oracle import rwkv7_ref as R
from rwkv_tl_amd import HIPGraph, RWKV7HIPBF16, State, make_rwkv7, sample_logits
from rwkv_tl_amd.checkpoint import make_random_state_dict
from rwkv_tl_amd.weight import RWKV7Weight

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
DEC_ATOL, DEC_RTOL, DEC_STATE = 1e-2, 8e-3, 1e-4
MM_ATOL, MM_RTOL, MM_STATE = DEC_ATOL, DEC_RTOL, DEC_STATE
REF_MAX_ABS = 4.0  # test/test_forward.py MAX_ABS_TOL


def tie(x: float) -> float:
    return 2e-2 + 2.0**-5 * abs(x)


def _rel(x, y):
    return float((x.double() - y.double()).norm() / y.double().norm().clamp_min(1e-30))


class BfSetup:
    def __init__(self, shape: str, cuda):
        self.sd = make_random_state_dict(shape, seed=0, dtype=BF)
        self.w = RWKV7Weight.from_state_dict(self.sd, device=cuda, dtype=BF)
        self.model = RWKV7HIPBF16(self.w, is_torch_compile=False)
        emb = self.w.emb.cpu()
        self.ref32 = R.Weights.from_emb(self.sd, emb, torch.float32)
        self.refbf = R.Weights.from_emb(self.sd, emb, BF)
        self.V = self.w.head.shape[0]


_CACHE: dict[str, BfSetup] = {}


def setup_for(shape, cuda) -> BfSetup:
    if shape not in _CACHE:
        _CACHE.clear()
        _CACHE[shape] = BfSetup(shape, cuda)
    return _CACHE[shape]


def _check_logits(got, ref, atol, rtol, label):
    got, ref = got.float().cpu(), ref.float().cpu()
    bad = (got - ref).abs() > atol + rtol * ref.abs()
    assert not bool(bad.any()), f"{label}: {int(bad.sum())} logits off, max |d|={(got - ref).abs().max():.3e}"


def _check_ref_semantics(got, ref, label):
    """The reference's bf16 criterion (test/test_forward.py:71-81)."""
    got, ref = got.float().cpu().reshape(-1), ref.float().cpu().reshape(-1)
    d = float((got - ref).abs().max())
    assert d <= REF_MAX_ABS, f"{label}: max |d|={d}"
    ga = int(got.argmax())
    top = float(ref.max())
    assert top - float(ref[ga]) <= tie(top), f"{label}: argmax {ga} vs {int(ref.argmax())}"
    top_got, top_ref = torch.topk(got, 5).indices, torch.topk(ref, 5)
    fifth = float(top_ref.values[-1])
    for i in set(top_got.tolist()) ^ set(top_ref.indices.tolist()):
        assert abs(float(ref[i]) - fifth) <= tie(fifth), f"{label}: top-5 differs at {i} beyond a near-tie"


def _check_state(S: State, ref, rel_bar, label):
    for i in range(len(S.tmix)):
        r = _rel(S.tmix[i]["rnn"].cpu(), ref[0][i]["rnn"])
        assert r < rel_bar, f"{label}: layer {i} rnn rel err {r:.2e}"
        xt = (S.tmix[i]["x"].cpu().float() - ref[0][i]["x"].float()).abs().max()
        xc = (S.cmix[i]["x"].cpu().float() - ref[1][i]["x"].float()).abs().max()
        assert xt <= 8e-2 and xc <= 8e-2, f"{label}: layer {i} shift state off ({xt:.2e}, {xc:.2e})"


@pytest.mark.parametrize("shape,steps", [("tiny", 24), ("0.1b", 48), ("0.4b", 32)])
def test_bf16_decode_matches_oracle(shape, steps, cuda):
    print(f"bf16 decode parity {shape} steps={steps}", flush=True)
    st = setup_for(shape, cuda)
    assert st.model.decode_launches(1) == 1, "bf16 batch-1 decode runs in the persistent kernel"
    g = torch.Generator().manual_seed(91)
    toks = torch.randint(0, st.V, (steps,), generator=g)
    S = st.model.new_state()
    assert S.tmix[0]["x"].dtype == BF
    s32 = R.new_state(st.w.L, st.w.C, dtype=BF)
    sbf = R.new_state(st.w.L, st.w.C, dtype=BF)
    errors0 = st.model.last_error()
    for i, t in enumerate(toks):
        lg, S = st.model.decode(t.reshape(1).to(cuda), S)
        assert lg.dtype == BF
        l32, s32 = R.decode(st.ref32, t.reshape(1), s32)
        lbf, sbf = R.decode(st.refbf, t.reshape(1), sbf)
        _check_logits(lg, l32, DEC_ATOL, DEC_RTOL, f"{shape} step {i} vs ref32")
        if i % 8 == 0 or i == steps - 1:
            _check_ref_semantics(lg, lbf, f"{shape} step {i} vs refbf")
    _check_state(S, s32, DEC_STATE, f"{shape} state vs ref32")
    assert st.model.last_error() == errors0


def test_bf16_multi_launch_decode_matches_persistent(cuda):
    """The GEMV path of a bf16 model (decode_path "kernels") against the
    persistent kernel and ref32."""
    st = setup_for("0.1b", cuda)
    g = torch.Generator().manual_seed(92)
    toks = torch.randint(0, st.V, (8,), generator=g)
    Sa, Sb = st.model.new_state(), st.model.new_state()
    s32 = R.new_state(st.w.L, st.w.C, dtype=BF)
    for i, t in enumerate(toks):
        la, Sa = st.model.decode(t.reshape(1).to(cuda), Sa)
        st.model.decode_path = "kernels"
        try:
            assert st.model.decode_launches(1) > 1
            lb, Sb = st.model.decode(t.reshape(1).to(cuda), Sb)
        finally:
            st.model.decode_path = "auto"
        l32, s32 = R.decode(st.ref32, t.reshape(1), s32)
        _check_logits(lb, l32, DEC_ATOL, DEC_RTOL, f"kernels step {i} vs ref32")
        _check_logits(lb, la, DEC_ATOL, DEC_RTOL, f"kernels step {i} vs persistent")
    _check_state(Sb, s32, DEC_STATE, "kernels state vs ref32")


@pytest.mark.slow
def test_bf16_large_m_prefill_matches_oracle(cuda):
    """A bf16 prefill long enough for the large-M GEMM path (0.4B, 2 x 1024 =
    2048 rows: hipBLASLt for the plain GEMMs, the large-M kernel for relu2,
    operands rounded to bf16): row 0's wkv state after the prefill against
    ref32's prefill of that sequence, within 4e-2 relative (the float16
    large-M bar of 5e-3 scaled by bf16's 2^3 coarser rounding), and the next
    decode's logits against the reference's own bf16 semantics with its
    criterion."""
    print("bf16 large-M prefill 0.4b 2x1024", flush=True)
    st = setup_for("0.4b", cuda)
    assert not st.model.f32_activations(2, 1024)
    g = torch.Generator().manual_seed(1024)
    prompt = torch.randint(0, st.V, (2, 1024), generator=g)
    nxt = torch.randint(0, st.V, (1, 2), generator=g)
    S = st.model.new_state(batch=2)
    st.model.prefill(prompt.to(cuda), S)
    s32 = R.new_state(st.w.L, st.w.C, dtype=BF)
    R.prefill(st.ref32, prompt[0], s32)
    for i in range(st.w.L):
        r = _rel(S.tmix[i]["rnn"][0].cpu(), s32[0][i]["rnn"])
        assert r < 4e-2, f"layer {i}: 2x1024 bf16 prefill row 0 vs ref32: {r:.2e}"
    lg, _ = st.model.decode(nxt[0].to(cuda), S)
    sbf = R.new_state(st.w.L, st.w.C, dtype=BF)
    R.prefill(st.refbf, prompt[0], sbf)
    lbf, _ = R.decode(st.refbf, nxt[0, :1], sbf)
    _check_ref_semantics(lg[0], lbf, "0.4b 2x1024 bf16 prefill + decode row 0 vs refbf")


@pytest.mark.parametrize("shape,B,T", [("tiny", 1, 40), ("0.1b", 2, 33), ("0.4b", 1, 128)])
def test_bf16_prefill_then_decode_matches_oracle(shape, B, T, cuda):
    print(f"bf16 prefill parity {shape} {B}x{T}", flush=True)
    st = setup_for(shape, cuda)
    g = torch.Generator().manual_seed(93 + T)
    prompt = torch.randint(0, st.V, (B, T), generator=g)
    nxt = torch.randint(0, st.V, (4, B), generator=g)
    S = st.model.new_state(batch=B)
    st.model.prefill(prompt.to(cuda), S)
    s32 = R.new_state(st.w.L, st.w.C, dtype=BF, batch=B)
    R.prefill(st.ref32, prompt, s32)
    _check_state(S, s32, MM_STATE, f"{shape} {B}x{T} prefill state vs ref32")
    for i in range(nxt.shape[0]):
        lg, S = st.model.decode(nxt[i].to(cuda), S)
        l32, s32 = R.decode(st.ref32, nxt[i], s32)
        for b in range(B):
            _check_logits(lg[b], l32[b], MM_ATOL, MM_RTOL, f"{shape} {B}x{T} decode {i} row {b} vs ref32")
    # the reference's bf16 semantics on row 0 after the prefill (one fresh decode)
    sbf = R.new_state(st.w.L, st.w.C, dtype=BF)
    R.prefill(st.refbf, prompt[0], sbf)
    lbf, _ = R.decode(st.refbf, nxt[0, :1], sbf)
    S0 = st.model.new_state()
    st.model.prefill(prompt[0].to(cuda), S0)
    lg0, _ = st.model.decode(nxt[0, :1].to(cuda), S0)
    _check_ref_semantics(lg0, lbf, f"{shape} 1x{T} prefill + decode vs refbf")


def test_bf16_batched_decode_rows_match_single_sequences(cuda):
    st = setup_for("tiny", cuda)
    B = 5
    g = torch.Generator().manual_seed(94)
    toks = torch.randint(0, st.V, (6, B), generator=g)
    SB = st.model.new_state(batch=B)
    singles = [st.model.new_state() for _ in range(B)]
    for i in range(toks.shape[0]):
        lgB, SB = st.model.decode(toks[i].to(cuda), SB)
        for b in range(B):
            lgb, singles[b] = st.model.decode(toks[i, b : b + 1].to(cuda), singles[b])
            _check_logits(lgB[b], lgb, MM_ATOL, MM_RTOL, f"B={B} step {i} row {b} vs B=1")


def test_bf16_graph_replay_and_factory(cuda):
    """make_rwkv7(backend="bf16") gives the bf16 class; HIP-graph replay of the
    multi-launch decode and of a prefill equals the eager calls bit for bit;
    the sampler reads bf16 logits directly."""
    st = setup_for("tiny", cuda)
    cls = make_rwkv7(torch.device("cuda"), backend="bf16", use_graph=False)
    assert cls is RWKV7HIPBF16
    with pytest.raises(ValueError, match="does not match"):
        RWKV7HIPBF16(RWKV7Weight.from_state_dict(make_random_state_dict("tiny", seed=0), device=cuda))
    st.model.decode_path = "kernels"
    try:
        graphed = HIPGraph(st.model)
        g = torch.Generator().manual_seed(95)
        prompt = torch.randint(0, st.V, (12,), generator=g)
        steps = torch.randint(0, st.V, (5,), generator=g)
        Sa, Sb = st.model.new_state(), st.model.new_state()
        graphed.prefill(prompt.to(cuda), Sa)
        st.model.prefill(prompt.to(cuda), Sb)
        for i, t in enumerate(steps):
            la, Sa = graphed.decode(t.reshape(1).to(cuda), Sa)
            torch.cuda.synchronize()
            lb, Sb = st.model.decode(t.reshape(1).to(cuda), Sb)
            assert torch.equal(la, lb), f"replay {i}"
        for x, y in zip(Sa.arenas, Sb.arenas):
            assert torch.equal(x, y)
    finally:
        st.model.decode_path = "auto"
    lg = la.reshape(1, -1)
    assert lg.dtype == BF
    assert int(sample_logits(lg)[0]) == int(lg.float().argmax())


def test_auto_backend_runs_bf16_weights(cuda):
    """make_rwkv7(dev, backend="auto") on bf16 weights: the reference returns
    RWKV7BF16 on every GPU of sm >= 80 (demo/__init__.py:98-104), so a caller
    who loads bfloat16 weights and passes "auto" gets a model that takes them.
    Its graph-wrapped decode follows the same model's eager decode bit for bit
    and the fp32 oracle at the batch-1 bar."""
    st = setup_for("tiny", cuda)
    cls = make_rwkv7(torch.device("cuda"), backend="auto")
    model = cls(st.w)
    assert isinstance(model.model, RWKV7HIPBF16)
    g = torch.Generator().manual_seed(7)
    toks = torch.randint(0, st.V, (6,), generator=g)
    S = model.new_state()
    Sr = st.model.new_state()
    sref = R.new_state(st.w.L, st.w.C, dtype=BF)
    for i, t in enumerate(toks):
        lg, S = model.decode(t.reshape(1).to(cuda), S)
        le, Sr = st.model.decode(t.reshape(1).to(cuda), Sr)
        assert lg.dtype == BF
        assert torch.equal(lg, le), f"graph vs eager, step {i}"
        lr, sref = R.decode(st.ref32, t.reshape(1), sref)
        _check_logits(lg, lr, DEC_ATOL, DEC_RTOL, f"auto step {i}")
