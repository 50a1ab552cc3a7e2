"""Parity of the HIP path at the 0.4B configurations the benchmark quotes.

* C4: 0.4B fp16 prefill for B x T in {1x8, 1x32, 1x64, 1x128, 1x512, 8x8,
  16x16} (real batches: B independent sequences of T tokens), zero initial
  state, then decode steps from the prefilled state -- the cases of the
  reference benchmark (script/benchmark_rwkv7.py:185-192), which flattens the
  batch into one sequence.
* C3: 0.4B decode at batch 16 from zero state, 256 steps.

Oracles as in test_gpu_model.py: ``ref32`` (fp32 math on the same fp16
weights, fp16 shift state) and ``ref16`` (the reference's fp16 semantics).
Bars, written where they are applied: logits within 1e-2 abs + 1e-3 rel
against both oracles at every checked step; per-layer wkv state of every row
within 1e-4 relative of ref32 after prefill and after the decode steps (the
every one of these steps keeps fp32-grade activations, the
batched GEMMs and the few-row kernel multiplying f32 activations as f16 parts
plus f16 remainders).

Decode steps: 64 after every prefill (C4 as stated) and 256 for C3. ref32
follows every row at every step through ``decode_rows`` (all rows in the same
torch operations, pinned to the row-by-row oracle in test_oracle.py); logits
are compared at every step of C4 and every 16th step (and the last) of C3.
ref16 is compared on rows 0 and B-1 at the first decode step: for C4 through
the committed fixture
``tests/golden/c4_ref16.safetensors`` (the oracle's fp16 path takes minutes per
128-token prefill on a CPU without fast half precision, so
``tests/golden/make_c4_ref16.py`` computed those logits -- the 64 largest and
2048 seeded random entries per row -- in the build container), for C3 live.
"""

from __future__ import annotations

import pytest
import torch

from safetensors.torch import load_file

from oracle import rwkv7_ref as R
from rwkv_tl_amd import RWKV7HIP, State
from rwkv_tl_amd.checkpoint import make_random_state_dict
from rwkv_tl_amd.weight import RWKV7Weight

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

LOGIT_ATOL, LOGIT_RTOL = 1e-2, 1e-3
STATE_REL = 1e-4

C4_CASES = [(1, 8), (1, 32), (1, 64), (1, 128), (1, 512), (8, 8), (16, 16)]


def _rel(x, y):
    return float((x.double() - y.double()).norm() / y.double().norm().clamp_min(1e-30))


def _check_logits(got, ref, label):
    got = got.float().cpu()
    ref = ref.float().cpu()
    bad = (got - ref).abs() > LOGIT_ATOL + LOGIT_RTOL * ref.abs()
    assert not bool(bad.any()), f"{label}: {int(bad.sum())} logits off, max |d|={(got - ref).abs().max():.3e}"


def _check_state(S: State, ref, rel_bar, label):
    """Every layer of every row: wkv state relative error, shift states abs."""
    for i in range(len(S.tmix)):
        r = _rel(S.tmix[i]["rnn"].cpu(), ref[0][i]["rnn"])
        assert r < rel_bar, f"{label}: layer {i} rnn rel err {r:.2e}"
        xt = (S.tmix[i]["x"].cpu().float() - ref[0][i]["x"].float()).abs().max()
        xc = (S.cmix[i]["x"].cpu().float() - ref[1][i]["x"].float()).abs().max()
        assert xt <= 2e-2 and xc <= 2e-2, f"{label}: layer {i} shift state off ({xt:.2e}, {xc:.2e})"


class Setup04:
    def __init__(self, cuda):
        sd = make_random_state_dict("0.4b", seed=0, dtype=torch.float16)
        self.w = RWKV7Weight.from_state_dict(sd, device=cuda, dtype=torch.float16)
        self.model = RWKV7HIP(self.w, is_torch_compile=False)
        emb = self.w.emb.cpu()
        self.ref32 = R.Weights.from_emb(sd, emb, torch.float32)
        self.ref16 = R.Weights.from_emb(sd, emb, torch.float16)
        self.V = self.w.head.shape[0]


@pytest.fixture(scope="module")
def m04(cuda):
    return Setup04(cuda)


def _run_decode_steps(m, S, s32, toks, label, check16, every=1):
    """Decode ``toks`` [steps, B] on the GPU and in ref32 (all rows at once),
    checking every row's logits against ref32 at every ``every``-th step and
    the last; ``check16(lg)`` checks the first step against ref16."""
    steps, B = toks.shape
    for i in range(steps):
        lg, S = m.model.decode(toks[i].to(m.w.device), S)
        l32, s32 = R.decode_rows(m.ref32, toks[i], s32)
        assert lg.shape == (B, m.V)
        if i % every == 0 or i == steps - 1:
            for b in range(B):
                _check_logits(lg[b], l32[b], f"{label} step {i} row {b} vs ref32")
        if i == 0:
            check16(lg)
        if i % 16 == 15:
            print(f"  {label}: {i + 1} decode steps checked", flush=True)
    return S, s32


@pytest.fixture(scope="module")
def c4_ref16(golden_dir):
    return load_file(str(golden_dir / "c4_ref16.safetensors"))


@pytest.mark.parametrize("B,T", C4_CASES, ids=[f"{b}x{t}" for b, t in C4_CASES])
def test_c4_prefill_then_decode_0p4b(m04, c4_ref16, B, T):
    steps = 64
    label = f"C4 0.4b {B}x{T}"
    print(f"{label}: prefill then {steps} decode steps", flush=True)
    g = torch.Generator().manual_seed(1000 * B + T)
    prompt = torch.randint(0, m04.V, (B, T), generator=g)
    toks = torch.randint(0, m04.V, (steps, B), generator=g)

    S = State(m04.w.L, m04.w.C, 64, device=m04.w.device, batch=B)
    m04.model.prefill(prompt.to(m04.w.device), S)
    s32 = R.new_state(m04.w.L, m04.w.C, dtype=torch.float16, batch=B)
    R.prefill(m04.ref32, prompt, s32)
    assert m04.model.f32_activations(B, T), "C4 prefills keep f32 activations"
    _check_state(S, s32, STATE_REL, f"{label} state after prefill vs ref32")
    print(f"  {label}: prefill state checked against ref32", flush=True)

    def check16(lg):
        for b in sorted({0, B - 1}):
            key = f"{B}x{T}_row{b}"
            assert c4_ref16[f"{key}_prompt_ends"].tolist() == [int(prompt[b, 0]), int(prompt[b, -1])], key
            idx = c4_ref16[f"{key}_idx"]
            _check_logits(lg[b].float().cpu()[idx], c4_ref16[f"{key}_val"], f"{label} step 0 row {b} vs ref16")

    S, s32 = _run_decode_steps(m04, S, s32, toks, label, check16)
    _check_state(S, s32, STATE_REL, f"{label} state after {steps} decode steps vs ref32")


def test_c3_decode_batch16_0p4b(m04):
    B, steps = 16, 256
    label = "C3 0.4b decode B=16"
    print(f"{label}: {steps} steps from zero state", flush=True)
    g = torch.Generator().manual_seed(316)
    toks = torch.randint(0, m04.V, (steps, B), generator=g)
    S = State(m04.w.L, m04.w.C, 64, device=m04.w.device, batch=B)
    s32 = R.new_state(m04.w.L, m04.w.C, dtype=torch.float16, batch=B)

    def check16(lg):
        for b in (0, B - 1):
            l16, _ = R.decode(m04.ref16, toks[0, b : b + 1], R.new_state(m04.w.L, m04.w.C, dtype=torch.float16))
            _check_logits(lg[b], l16, f"{label} step 0 row {b} vs ref16")

    S, s32 = _run_decode_steps(m04, S, s32, toks, label, check16, every=16)
    _check_state(S, s32, STATE_REL, f"{label} state after {steps} steps vs ref32")
