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


def _brute_loss(S, ins, gy, gS):
    """L = <gy, y> + <gS, S_T> of wkv7_brute (pure-Python doubles); S [H,N,N],
    ins six [T,H,N] nested lists."""
    ys, ST = R.wkv7_brute(S, *ins)
    L = 0.0
    for t, yt in enumerate(ys):
        for h, yh in enumerate(yt):
            L += sum(yv * g for yv, g in zip(yh, gy[t][h]))
    for h, Sh in enumerate(ST):
        for i, row in enumerate(Sh):
            L += sum(x * g for x, g in zip(row, gS[h][i]))
    return L


def test_wkv7_scan_grads_match_finite_differences():
    """The oracle's DPLR gradients (torch autograd of the fp32 serial scan)
    against central differences of the pure-Python double-precision loop, in
    random directions through every input (S0, r, w, k, v, a, b)."""
    g = torch.Generator().manual_seed(11)
    H, N, T = 2, 4, 3
    S = torch.randn(H, N, N, generator=g, dtype=torch.float64) * 0.5
    ins = [torch.randn(T, H, N, generator=g, dtype=torch.float64) * 0.5 for _ in range(6)]
    ins[1] = torch.rand(T, H, N, generator=g, dtype=torch.float64) * 0.5 + 0.45  # w in (0.45, 0.95)
    gy = torch.randn(T, H, N, generator=g, dtype=torch.float64)
    gS = torch.randn(H, N, N, generator=g, dtype=torch.float64)
    # argument order of wkv7_brute / wkv7_scan: r, w, k, v, a, b
    grads = R.wkv7_scan_grads(S.unsqueeze(0), *(x.unsqueeze(0) for x in ins), gy.unsqueeze(0), gS.unsqueeze(0))
    eps = 1e-6
    for trial in range(4):
        dirs = [torch.randn(x.shape, generator=g, dtype=torch.float64) for x in [S] + ins]
        def at(sign):
            S2 = (S + sign * eps * dirs[0]).tolist()
            i2 = [(x + sign * eps * d).tolist() for x, d in zip(ins, dirs[1:])]
            return _brute_loss(S2, i2, gy.tolist(), gS.tolist())
        fd = (at(1) - at(-1)) / (2 * eps)
        an = sum(float((gr.double().reshape(d.shape) * d).sum()) for gr, d in zip(grads, dirs))
        assert abs(fd - an) <= 1e-4 * max(1.0, abs(fd)), f"trial {trial}: finite difference {fd} vs autograd {an}"


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


# --------------------------------------------------------------------------
# Operator-level oracle (the time-mix stages one by one)
# --------------------------------------------------------------------------


def test_operator_oracle_composes_to_time_mix():
    """One token of ``time_mix`` (pinned by the reference's golden vectors)
    rebuilt from the operator restatements: rank_gemv -> gates -> l2norm_neg_kk_a
    -> wkv7_step -> gn_rkrk -> gate and o-projection. A dropped term, a wrong
    operand or a swapped activation in any operator breaks the match."""
    sd = make_random_state_dict("tiny", seed=3, dtype=torch.float32)
    W = R.Weights(sd, dtype=torch.float32)
    H, C, N = W.H, W.C, 64
    att = W.blocks[1].att
    g = torch.Generator().manual_seed(11)
    x0, prev, v_first = (torch.randn(C, generator=g) for _ in range(3))
    S0 = torch.randn(H, N, N, generator=g) * 0.1
    st = {"x": prev.clone(), "rnn": S0.clone()}
    out_ref, _ = R.time_mix(att, x0, v_first.clone(), st, H, N)

    x = att.ln_pre(x0)
    xr, xw, xk, xv, xa, xg = (x + getattr(att, n) * (prev - x) for n in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"))
    r, k, v = xr @ att.rkvWt[0], xk @ att.rkvWt[1], xv @ att.rkvWt[2]
    ranks = [att.v1.shape[1], att.w1.shape[1], att.a1.shape[1], att.g1.shape[1]]
    packed = torch.cat([att.v1.t(), att.w1.t(), att.a1.t(), att.g1.t()])
    vr, wr, ar, gr = R.rank_gemv(xv, xw, xa, xg, packed, *ranks).split(ranks)
    vec = lambda t: t.reshape(-1)  # noqa: E731
    v2, w2, a, kk, k2, gg = R.gates(vr, wr, ar, gr, v, v_first, k, att.v2.t(), att.w2.t(), att.a2.t(), att.g2.t(),
                                    vec(att.v0), vec(att.w0), vec(att.a0), vec(att.k_k), vec(att.k_a))
    kn, b = R.l2norm_neg_kk_a(kk.reshape(H, N), a.reshape(H, N))
    hn = lambda t: t.reshape(H, N)  # noqa: E731
    y, S1 = R.wkv7_step(S0, hn(r), hn(w2), hn(k2), hn(v2), kn, b)
    yo = R.gn_rkrk(y, hn(r), hn(k2), hn(v2), att.r_k, att.ln_x.w, att.ln_x.b)
    out = x0 + (yo * gg) @ att.oWt
    torch.testing.assert_close(out, out_ref, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(S1, st["rnn"], rtol=1e-5, atol=1e-6)


def test_operator_oracle_closed_forms():
    """Limits and special points that fix each formula."""
    e = math.exp
    C = 8
    z, one = torch.zeros(C), torch.ones(C)
    big = torch.full((C,), 80.0)
    sq = math.sqrt(math.e)
    torch.testing.assert_close(R.w_gate(z, z), torch.full((C,), e(-0.5 / sq)))
    torch.testing.assert_close(R.w_gate(big, z), torch.full((C,), e(-1 / sq)))
    torch.testing.assert_close(R.w_gate(-big, z), one)
    v, vf = torch.arange(C, dtype=torch.float32), -torch.arange(C, dtype=torch.float32) - 1
    torch.testing.assert_close(R.v_gate(v, vf, -big, z), v)
    torch.testing.assert_close(R.v_gate(v, vf, big, z), vf)
    torch.testing.assert_close(R.v_gate(v, vf, z, z), (v + vf) / 2)
    k, kk_ = torch.linspace(-2, 2, C), torch.linspace(0.5, 1.5, C)
    a, kk, k0 = R.a_kk_k(z, z, k, kk_, z)
    torch.testing.assert_close(a, one / 2)
    torch.testing.assert_close(kk, k * kk_)
    torch.testing.assert_close(k0, k)  # k_a = 0 keeps k
    _, _, k1 = R.a_kk_k(z, z, k, kk_, one)
    torch.testing.assert_close(k1, k * 0.5)  # k_a = 1 gives k * a
    # L2 norm: unit rows, the zero row stays zero (clamp at 1e-12), b = -kn * a
    H = 3
    kkh = torch.randn(H, 64, generator=torch.Generator().manual_seed(2))
    kkh[1] = 0
    ah = torch.rand(H, 64, generator=torch.Generator().manual_seed(3))
    kn, b = R.l2norm_neg_kk_a(kkh, ah)
    torch.testing.assert_close(kn.norm(dim=1), torch.tensor([1.0, 0.0, 1.0]))
    torch.testing.assert_close(b, -kn * ah)
    # GroupNorm: a constant head normalises to 0 (out = ln_b + rk * v); a head
    # 0..63 has mean 31.5 and biased variance (64^2 - 1) / 12
    y = torch.stack([torch.full((64,), 5.0), torch.arange(64, dtype=torch.float32)])
    r_, k_, v_, rk_ = (torch.rand(2, 64, generator=torch.Generator().manual_seed(s)) for s in (4, 5, 6, 7))
    lw, lb = torch.rand(128, generator=torch.Generator().manual_seed(8)), torch.rand(128, generator=torch.Generator().manual_seed(9))
    out = R.gn_rkrk(y, r_, k_, v_, rk_, lw, lb).reshape(2, 64)
    bonus = (r_ * k_ * rk_).sum(1, keepdim=True) * v_
    torch.testing.assert_close(out[0], lb[:64] + bonus[0])
    yn = (torch.arange(64.0) - 31.5) / math.sqrt((64 * 64 - 1) / 12 + 64e-5)
    torch.testing.assert_close(out[1], yn * lw[64:] + lb[64:] + bonus[1])
    # rank_gemv: a one-hot row j selects element j of its segment's input
    rv, rw, ra, rg, Cx = 2, 3, 1, 2, 8
    xs = [torch.randn(Cx, generator=torch.Generator().manual_seed(20 + i)) for i in range(4)]
    packed = torch.zeros(rv + rw + ra + rg, Cx)
    for j in range(rv + rw + ra + rg):
        packed[j, j] = 1.0
    seg = [0] * rv + [1] * rw + [2] * ra + [3] * rg
    torch.testing.assert_close(R.rank_gemv(*xs, packed, rv, rw, ra, rg), torch.stack([xs[seg[j]][j] for j in range(8)]))
    # gates with zero second-step matrices: v12 = w12 = a12 = g12 = 0
    Rk = 4
    zr, zm = torch.zeros(Rk), torch.zeros(C, Rk)
    v0_, w0_, a0_ = torch.linspace(-1, 1, C), torch.linspace(-2, 2, C), torch.linspace(-3, 3, C)
    vo, wo, ao, kko, ko, go = R.gates(zr, zr, zr, zr, v, vf, k, zm, zm, zm, zm, v0_, w0_, a0_, kk_, one)
    torch.testing.assert_close(vo, v + torch.sigmoid(v0_) * (vf - v))
    torch.testing.assert_close(wo, torch.exp(-torch.sigmoid(w0_) / sq))
    torch.testing.assert_close(ao, torch.sigmoid(a0_))
    torch.testing.assert_close(ko, k * torch.sigmoid(a0_))
    torch.testing.assert_close(go, z)


@pytest.mark.slow
def test_c4_ref16_fixture_matches_oracle(golden_dir):
    """The committed C4 fp16-oracle fixture (tests/golden/make_c4_ref16.py) is
    the oracle's own output: recompute the 1x8 case here and compare the stored
    entries exactly; the stored indices include the 64 largest logits."""
    from safetensors.torch import load_file

    from rwkv_tl_amd.weight import RWKV7Weight

    fx = load_file(str(golden_dir / "c4_ref16.safetensors"))
    sd = make_random_state_dict("0.4b", seed=0, dtype=torch.float16)
    w = RWKV7Weight.from_state_dict(sd, device="cpu", dtype=torch.float16)
    W16 = R.Weights.from_emb(sd, w.emb, torch.float16)
    V = w.head.shape[0]
    g = torch.Generator().manual_seed(1000 * 1 + 8)
    prompt = torch.randint(0, V, (1, 8), generator=g)
    toks = torch.randint(0, V, (64, 1), generator=g)
    assert fx["1x8_row0_prompt_ends"].tolist() == [int(prompt[0, 0]), int(prompt[0, -1])]
    st = R.new_state(w.L, w.C, dtype=torch.float16)
    R.prefill(W16, prompt[0], st)
    lg, _ = R.decode(W16, toks[0, :1], st)
    idx = fx["1x8_row0_idx"]
    assert torch.equal(lg.float()[idx], fx["1x8_row0_val"])
    assert set(torch.topk(lg.float(), 64).indices.tolist()) == set(idx[:64].tolist())


@pytest.mark.parametrize("shape", ["tiny", "0.1b"])
def test_decode_rows_matches_row_by_row_decode(shape):
    """``decode_rows`` (all rows of a batched state in the same torch ops, the
    fast checker of the batched GPU tests) equals ``decode`` (each row as its
    own single-sequence state, golden-pinned) on fp32 weights: logits and wkv
    states to fp32 rounding over 6 steps of 5 rows from a non-zero state, the
    f16 shift states to one half-precision step."""
    from rwkv_tl_amd.checkpoint import make_random_state_dict

    sd = make_random_state_dict(shape, seed=0, dtype=torch.float16)
    W = R.Weights(sd, torch.float32)
    B = 5
    g = torch.Generator().manual_seed(8)
    toks = torch.randint(0, W.head.shape[0], (7, B), generator=g)
    sa = R.new_state(W.L, W.C, dtype=torch.float16, batch=B)
    R.decode(W, toks[0], sa)  # a non-zero starting state
    sb = ([{k: v.clone() for k, v in d.items()} for d in sa[0]], [{k: v.clone() for k, v in d.items()} for d in sa[1]])
    for i in range(1, 7):
        la, sa = R.decode(W, toks[i], sa)
        lb, sb = R.decode_rows(W, toks[i], sb)
        torch.testing.assert_close(lb, la, rtol=1e-5, atol=1e-5)
    for i in range(W.L):
        for b in range(B):
            x, y = sb[0][i]["rnn"][b].double(), sa[0][i]["rnn"][b].double()
            assert float((x - y).norm() / y.norm()) < 1e-5, f"layer {i} row {b}"
        for part in (0, 1):
            torch.testing.assert_close(sb[part][i]["x"].float(), sa[part][i]["x"].float(), rtol=0, atol=2e-3)
