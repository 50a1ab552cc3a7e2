"""Batch-1 decode on int8 weights (``RWKV7HIP(weight_quant="int8")``) on the GPU.

The int8 decode streams per-row symmetric int8 copies of the layer matrices
(receptance/key/value, LoRA first steps, output, FFN key/value) and of the
head, with f32 row scales applied to the f32 dot products. Its oracle is the
fp32-math model (``ref32``) on the DEQUANTIZED weights ``scale[n] * q[n, :]``,
built here from the same seed-0 checkpoint: the kernel then differs from the
oracle only by summation order, so the fp16-decode bars apply unchanged --
logits within 1e-2 abs + 1e-3 rel at every step, fp32 wkv state within 1e-4
relative per layer at the end. A kernel that used a wrong row's scale, mixed
up the order of the LoRA rows or mis-addressed a section of the int8 arena
fails these by orders of magnitude (a test below also shows the fp16 model
misses the bar against the dequantized oracle, i.e. the bar does see the
quantisation).
"""

from __future__ import annotations

import pytest
import torch

from oracle import rwkv7_ref as R
from rwkv_tl_amd import RWKV7HIP, RWKV7HIPInt8, State, _lib
from rwkv_tl_amd.checkpoint import make_random_state_dict
from rwkv_tl_amd.weight import RWKV7Weight, pack_device_weights, quantize_rows_i8

pytestmark = pytest.mark.gpu

LOGIT_ATOL, LOGIT_RTOL = 1e-2, 1e-3
STATE_REL = 1e-4


def _rel(x, y):
    return float((x.double() - y.double()).norm() / y.double().norm().clamp_min(1e-30))


def dequantized_state_dict(sd: dict[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    """The checkpoint with every int8-streamed matrix replaced by
    ``scale * q`` (fp32), rows taken in the ``[out, in]`` orientation the
    decode dots run over (the LoRA first steps ``[C, R]`` are quantised per
    column, i.e. per row of their transpose)."""
    out = dict(sd)

    def deq_rows(W):
        q, s = quantize_rows_i8(W)
        return q.float() * s[:, None]

    for k, v in sd.items():
        if k == "head.weight" or k.endswith(
            (".att.receptance.weight", ".att.key.weight", ".att.value.weight", ".att.output.weight",
             ".ffn.key.weight", ".ffn.value.weight")
        ):
            out[k] = deq_rows(v)
        elif any(k.endswith(f".att.{g}1") for g in "wavg"):
            out[k] = deq_rows(v.T).T.contiguous()
    return out


class Int8Setup:
    def __init__(self, shape: str, cuda):
        sd = make_random_state_dict(shape, seed=0, dtype=torch.float16)
        self.w = RWKV7Weight.from_state_dict(sd, device=cuda, dtype=torch.float16)
        self.model = RWKV7HIPInt8(self.w, is_torch_compile=False)
        emb = self.w.emb.cpu()
        self.ref32q = R.Weights.from_emb(dequantized_state_dict(sd), emb, torch.float32)
        self.ref32 = R.Weights.from_emb(sd, emb, torch.float32)
        self.V = self.w.head.shape[0]


_CACHE: dict[str, Int8Setup] = {}


def setup_for(shape, cuda) -> Int8Setup:
    if shape not in _CACHE:
        _CACHE.clear()
        _CACHE[shape] = Int8Setup(shape, cuda)
    return _CACHE[shape]


def _bad_logits(got, ref):
    got, ref = got.float().cpu(), ref.float().cpu()
    return int(((got - ref).abs() > LOGIT_ATOL + LOGIT_RTOL * ref.abs()).sum()), float((got - ref).abs().max())


def test_int8_arena_packed_on_the_gpu_equals_the_cpu_packing(cuda):
    """The GPU quantises the checkpoint to the same bytes as the CPU (the
    dequantized oracle above quantises on the CPU)."""
    st = setup_for("0.1b", cuda)
    sd = make_random_state_dict("0.1b", seed=0, dtype=torch.float16)
    wc = RWKV7Weight.from_state_dict(sd, device="cpu", dtype=torch.float16)
    cpu = pack_device_weights(wc, fragments=False, int8=True)
    assert torch.equal(st.model.dev.layers_q.cpu(), cpu.layers_q)
    assert torch.equal(st.model.dev.head_q.cpu(), cpu.head_q)


@pytest.mark.parametrize("shape,steps", [("tiny", 24), ("0.1b", 48), ("0.4b", 64)])
def test_int8_decode_matches_dequantized_oracle(shape, steps, cuda):
    print(f"int8 decode parity {shape} steps={steps}", flush=True)
    st = setup_for(shape, cuda)
    assert st.model.decode_launches(1) == 1, "int8 decode runs in the persistent kernel"
    g = torch.Generator().manual_seed(77)
    toks = torch.randint(0, st.V, (steps,), generator=g)
    S = State(st.w.L, st.w.C, 64, device=cuda)
    s32 = R.new_state(st.w.L, st.w.C, dtype=torch.float16)
    errors0 = st.model.last_error()
    for i, t in enumerate(toks):
        lg, S = st.model.decode(t.reshape(1).to(cuda), S)
        l32, s32 = R.decode(st.ref32q, t.reshape(1), s32)
        n, dmax = _bad_logits(lg, l32)
        assert n == 0, f"{shape} step {i}: {n} logits off the dequantized oracle, max |d|={dmax:.3e}"
    for i in range(st.w.L):
        r = _rel(S.tmix[i]["rnn"].cpu(), s32[0][i]["rnn"])
        assert r < STATE_REL, f"{shape}: layer {i} rnn rel err {r:.2e}"
        xt = (S.tmix[i]["x"].cpu().float() - s32[0][i]["x"].float()).abs().max()
        xc = (S.cmix[i]["x"].cpu().float() - s32[1][i]["x"].float()).abs().max()
        assert xt <= 2e-2 and xc <= 2e-2, f"{shape}: layer {i} shift state off ({xt:.2e}, {xc:.2e})"
    assert st.model.last_error() == errors0, "a persistent decode launch aborted"


def test_int8_bar_sees_the_quantisation(cuda):
    """The fp16-weight oracle and the dequantized oracle differ by far more
    than the bar, so the parity test above pins the int8 arithmetic."""
    st = setup_for("0.1b", cuda)
    g = torch.Generator().manual_seed(78)
    toks = torch.randint(0, st.V, (4,), generator=g)
    sa = R.new_state(st.w.L, st.w.C, dtype=torch.float16)
    sb = R.new_state(st.w.L, st.w.C, dtype=torch.float16)
    S = State(st.w.L, st.w.C, 64, device=cuda)
    for t in toks:
        la, sa = R.decode(st.ref32, t.reshape(1), sa)
        lb, sb = R.decode(st.ref32q, t.reshape(1), sb)
        lg, S = st.model.decode(t.reshape(1).to(cuda), S)
    assert _bad_logits(la, lb)[0] > 100
    assert _bad_logits(lg, la)[0] > 100, "the int8 kernel matches the fp16 oracle: int8 weights not streamed"
    assert _bad_logits(lg, lb)[0] == 0


def test_int8_model_batched_decode_and_prefill_use_f16(cuda):
    """Prefill and batched decode of an int8 model read the fp16 arenas: same
    results as the fp16 model, bit for bit."""
    st = setup_for("tiny", cuda)
    f16 = RWKV7HIP(st.w, is_torch_compile=False)
    g = torch.Generator().manual_seed(79)
    B, T = 3, 20
    prompt = torch.randint(0, st.V, (B, T), generator=g).to(cuda)
    nxt = torch.randint(0, st.V, (B,), generator=g).to(cuda)
    Sa = State(st.w.L, st.w.C, 64, device=cuda, batch=B)
    Sb = State(st.w.L, st.w.C, 64, device=cuda, batch=B)
    st.model.prefill(prompt, Sa)
    f16.prefill(prompt, Sb)
    la, Sa = st.model.decode(nxt, Sa)
    lb, Sb = f16.decode(nxt, Sb)
    assert torch.equal(la, lb)
    for x, y in zip(Sa.arenas, Sb.arenas):
        assert torch.equal(x, y)


def test_int8_decode_refuses_the_multi_launch_path(cuda):
    st = setup_for("tiny", cuda)
    st.model.decode_path = "kernels"
    try:
        S = State(st.w.L, st.w.C, 64, device=cuda)
        with pytest.raises(_lib.HipError, match="unsupported shape"):
            st.model.decode(torch.tensor([1], device=cuda), S)
    finally:
        st.model.decode_path = "auto"
