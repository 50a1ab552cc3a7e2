"""Pins of the CPU oracle (``oracle/rwkv7_ref.py``) -- CPU only.

1. Golden vectors written by the reference's own pure-torch path
   (``tests/golden/make_golden.py``): the restated model must reproduce them on
   the same seeded checkpoint (fp32 and fp16, decode / prefill / forward,
   logits and every state tensor), and config C1 (0.1B, 32 greedy steps).
2. The DPLR step against a pure-Python brute force on tiny inputs, and
   against closed forms the recurrence must satisfy.
3. The seeded checkpoint generator against the digests in the manifest.
"""

from __future__ import annotations

import json
import math

import pytest
import torch
from safetensors.torch import load_file

from oracle import rwkv7_ref as R
from rwkv_tl_amd.checkpoint import SHAPES, make_random_state_dict, state_dict_digest


def _tiny(dtype):
    sd = make_random_state_dict("tiny", seed=0, dtype=torch.float32)
    return R.Weights(sd, dtype)


@pytest.mark.parametrize("dtype,name", [(torch.float32, "tiny_fp32"), (torch.float16, "tiny_fp16")])
def test_oracle_matches_reference_golden(dtype, name, manifest, golden_dir):
    gold = load_file(str(golden_dir / f"{name}.safetensors"))
    toks = manifest["tiny"]["tokens"]
    W = _tiny(dtype)
    # LN0 of the embedding at load (weight.py:175)
    torch.testing.assert_close(W.emb[:32].float(), gold["emb_ln0_head"], rtol=0, atol=0)
    torch.testing.assert_close(W.emb.double().sum(1), gold["emb_ln0_rowsum"], rtol=0, atol=1e-9)

    st = R.new_state(W.L, W.C, dtype=dtype)
    logits = []
    for t in toks:
        lg, st = R.decode(W, torch.tensor([t]), st)
        logits.append(lg.float())
    torch.testing.assert_close(torch.stack(logits), gold["decode_logits"], rtol=0, atol=0)
    for i in range(W.L):
        torch.testing.assert_close(st[0][i]["rnn"], gold[f"decode_state.{i}.rnn"], rtol=0, atol=0)
        torch.testing.assert_close(st[0][i]["x"].float(), gold[f"decode_state.{i}.tmix_x"], rtol=0, atol=0)
        torch.testing.assert_close(st[1][i]["x"].float(), gold[f"decode_state.{i}.cmix_x"], rtol=0, atol=0)

    st = R.new_state(W.L, W.C, dtype=dtype)
    R.prefill(W, torch.tensor(toks[:-1]), st)
    for i in range(W.L):
        torch.testing.assert_close(st[0][i]["rnn"], gold[f"prefill_state.{i}.rnn"], rtol=0, atol=0)
        torch.testing.assert_close(st[0][i]["x"].float(), gold[f"prefill_state.{i}.tmix_x"], rtol=0, atol=0)
        torch.testing.assert_close(st[1][i]["x"].float(), gold[f"prefill_state.{i}.cmix_x"], rtol=0, atol=0)
    lg, _ = R.decode(W, torch.tensor([toks[-1]]), st)
    torch.testing.assert_close(lg.float(), gold["prefill_then_decode_logits"], rtol=0, atol=0)

    st = R.new_state(W.L, W.C, dtype=dtype)
    lg, _ = R.forward(W, torch.tensor(toks), st)
    torch.testing.assert_close(lg.float(), gold["forward_logits"], rtol=0, atol=0)


def test_checkpoint_generator_digest(manifest):
    sd = make_random_state_dict("tiny", seed=0, dtype=torch.float32)
    assert state_dict_digest(sd) == manifest["tiny"]["weights_fp32_sha256"]
    assert SHAPES["tiny"].__dict__ == manifest["tiny"]["shape"]


@pytest.mark.slow
def test_oracle_c1_greedy_decode(manifest, golden_dir):
    """Config C1: 0.1B fp32, prompt decoded token by token, 32 greedy steps."""
    c1 = json.loads((golden_dir / "c1_0p1b.json").read_text())
    sd = make_random_state_dict("0.1b", seed=0, dtype=torch.float32)
    assert state_dict_digest(sd) == manifest["c1"]["weights_fp32_sha256"]
    W = R.Weights(sd, torch.float32)
    del sd
    st = R.new_state(W.L, W.C, dtype=torch.float32)
    lg = None
    for t in c1["prompt"]:
        lg, st = R.decode(W, torch.tensor([t]), st)
    ids = []
    for step in c1["steps"]:
        top = torch.topk(lg, 5)
        assert top.indices.tolist() == step["top5_ids"]
        assert top.values.tolist() == pytest.approx(step["top5_vals"], abs=1e-5)
        assert float(lg.double().sum()) == pytest.approx(step["sum"], rel=1e-6, abs=1e-4)
        assert float(lg.double().norm()) == pytest.approx(step["l2"], rel=1e-6)
        nxt = int(lg.argmax())
        ids.append(nxt)
        lg, st = R.decode(W, torch.tensor([nxt]), st)
    assert ids == c1["greedy_ids"]
    for i in range(W.L):
        ref = c1["final_state"][f"layer{i}"]
        assert float(st[0][i]["rnn"].double().norm()) == pytest.approx(ref["rnn_l2"], rel=1e-6)
        assert float(st[0][i]["x"].double().norm()) == pytest.approx(ref["tmix_x_l2"], rel=1e-6)
        assert float(st[1][i]["x"].double().norm()) == pytest.approx(ref["cmix_x_l2"], rel=1e-6)


# ---------------------------------------------------------------------------
# DPLR step pins
# ---------------------------------------------------------------------------


def _rand_step(H=2, N=4, T=3, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    S = torch.randn(H, N, N, generator=g, dtype=dtype)
    vecs = [torch.randn(T, H, N, generator=g, dtype=dtype) for _ in range(6)]
    vecs[1] = torch.rand(T, H, N, generator=g, dtype=dtype)  # w in (0, 1)
    return S, vecs


def test_wkv7_step_matches_brute_force():
    S, (r, w, k, v, a, b) = _rand_step()
    Sf = S.float()
    ys = []
    for t in range(r.shape[0]):
        y, Sf = R.wkv7_step(Sf, r[t].float(), w[t].float(), k[t].float(), v[t].float(), a[t].float(), b[t].float())
        ys.append(y)
    yb, Sb = R.wkv7_brute(S.tolist(), r.tolist(), w.tolist(), k.tolist(), v.tolist(), a.tolist(), b.tolist())
    torch.testing.assert_close(torch.stack(ys).double(), torch.tensor(yb, dtype=torch.float64), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(Sf.double(), torch.tensor(Sb, dtype=torch.float64), rtol=1e-5, atol=1e-5)


def _steps(step, S, vecs):
    r, w, k, v, a, b = vecs
    ys = []
    for t in range(r.shape[0]):
        y, S = step(S, r[t], w[t], k[t], v[t], a[t], b[t])
        ys.append(y)
    return torch.stack(ys), S


def test_wkv7_brute_plants_detected():
    """Planted mistakes in a copy of the oracle's step (CPU only) must fail the
    brute-force check that the real step passes: the check can tell a wrong
    index, a dropped term, a wrong sign and a stale operand apart."""
    S, vecs = _rand_step(T=3, dtype=torch.float32)
    yb, Sb = R.wkv7_brute(S.tolist(), *[x.tolist() for x in vecs])
    yb, Sb = torch.tensor(yb, dtype=torch.float64), torch.tensor(Sb, dtype=torch.float64)

    def agrees(step):
        y, Sn = _steps(step, S.clone(), vecs)
        return torch.allclose(y.double(), yb, rtol=1e-5, atol=1e-6) and torch.allclose(
            Sn.double(), Sb, rtol=1e-5, atol=1e-6
        )

    assert agrees(R.wkv7_step)

    def decay_rows(S, r, w, k, v, a, b):  # w applied along the value axis
        Sn = S * w.unsqueeze(2) + torch.einsum("hva,ha,hb->hvb", S, a, b) + torch.einsum("hv,hk->hvk", v, k)
        return torch.einsum("hvk,hk->hv", Sn, r), Sn

    def no_rank1(S, r, w, k, v, a, b):  # dropped (S a) b^T
        Sn = S * w.unsqueeze(1) + torch.einsum("hv,hk->hvk", v, k)
        return torch.einsum("hvk,hk->hv", Sn, r), Sn

    def flipped(S, r, w, k, v, a, b):  # wrong sign on the rank-1 term
        Sn = S * w.unsqueeze(1) - torch.einsum("hva,ha,hb->hvb", S, a, b) + torch.einsum("hv,hk->hvk", v, k)
        return torch.einsum("hvk,hk->hv", Sn, r), Sn

    def stale_sa(S, r, w, k, v, a, b):  # S a taken after the decay instead of before
        Sd = S * w.unsqueeze(1)
        Sn = Sd + torch.einsum("hva,ha,hb->hvb", Sd, a, b) + torch.einsum("hv,hk->hvk", v, k)
        return torch.einsum("hvk,hk->hv", Sn, r), Sn

    def kv_swapped(S, r, w, k, v, a, b):  # k v^T instead of v k^T
        Sn = S * w.unsqueeze(1) + torch.einsum("hva,ha,hb->hvb", S, a, b) + torch.einsum("hk,hv->hvk", v, k)
        return torch.einsum("hvk,hk->hv", Sn, r), Sn

    def y_before(S, r, w, k, v, a, b):  # y read from the old state
        Sn = S * w.unsqueeze(1) + torch.einsum("hva,ha,hb->hvb", S, a, b) + torch.einsum("hv,hk->hvk", v, k)
        return torch.einsum("hvk,hk->hv", S, r), Sn

    for bad in (decay_rows, no_rank1, flipped, stale_sa, kv_swapped, y_before):
        assert not agrees(bad), bad.__name__


def test_wkv7_closed_forms():
    H, N, T = 2, 8, 5
    g = torch.Generator().manual_seed(3)
    k = torch.randn(1, T, H, N, generator=g, dtype=torch.float64)
    v = torch.randn(1, T, H, N, generator=g, dtype=torch.float64)
    r = torch.randn(1, T, H, N, generator=g, dtype=torch.float64)
    zero = torch.zeros_like(k)
    ones = torch.ones_like(k)
    # w = 1, a = b = 0: S_T = S_0 + sum_t v_t k_t^T and y_t = S_t r_t
    S0 = torch.randn(1, H, N, N, generator=g, dtype=torch.float64)
    y, ST = R.wkv7_scan(S0, r, ones, k, v, zero, zero)
    expect = S0[0] + torch.einsum("thv,thk->hvk", v[0], k[0])
    torch.testing.assert_close(ST[0].double(), expect, rtol=1e-6, atol=1e-6)
    S_t = S0[0] + torch.einsum("hv,hk->hvk", v[0, 0], k[0, 0])
    torch.testing.assert_close(y[0, 0].double(), torch.einsum("hvk,hk->hv", S_t, r[0, 0]), rtol=1e-6, atol=1e-6)
    # k = v = 0, a = 0: columns decay by the product of w
    w = torch.rand(1, T, H, N, generator=g, dtype=torch.float64)
    _, ST = R.wkv7_scan(S0, r, w, zero, zero, zero, zero)
    torch.testing.assert_close(ST[0].double(), S0[0] * w[0].prod(0).unsqueeze(1), rtol=1e-6, atol=1e-9)
    # linear in S: scan(S1 + S2) - scan(0) = (scan(S1) - scan(0)) + (scan(S2) - scan(0))
    a = torch.nn.functional.normalize(torch.randn(1, T, H, N, generator=g, dtype=torch.float64), dim=-1)
    b = -a * torch.rand(1, T, H, N, generator=g, dtype=torch.float64)
    S1 = torch.randn(1, H, N, N, generator=g, dtype=torch.float64)
    S2 = torch.randn(1, H, N, N, generator=g, dtype=torch.float64)
    run = lambda S: R.wkv7_scan(S, r, w, k, v, a, b)[1].double()  # noqa: E731
    base = run(torch.zeros_like(S1))
    torch.testing.assert_close(run(S1 + S2) - base, (run(S1) - base) + (run(S2) - base), rtol=1e-5, atol=1e-6)


def test_layernorm_closed_forms():
    """LN0/LN1/LN2 are F.layer_norm with eps 1e-5: check against its definition
    on a row whose mean and variance are known exactly."""
    C = 256
    x = torch.arange(C, dtype=torch.float64) - (C - 1) / 2  # mean 0, var (C^2-1)/12
    ln = R._LN({"p.weight": torch.ones(C, dtype=torch.float64), "p.bias": torch.zeros(C, dtype=torch.float64)}, "p")
    y = ln(x)
    torch.testing.assert_close(y, x / math.sqrt((C * C - 1) / 12 + 1e-5))
    const = torch.full((C,), 3.0, dtype=torch.float64)
    ln2 = R._LN({"p.weight": torch.ones(C, dtype=torch.float64), "p.bias": torch.full((C,), 0.5, dtype=torch.float64)}, "p")
    torch.testing.assert_close(ln2(const), torch.full((C,), 0.5, dtype=torch.float64))
