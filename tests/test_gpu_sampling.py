"""HIP sampling kernel (rwkv7_sample) against the CPU oracle (oracle/sampling_ref.py).

* Greedy, top-k=1 and penalties: exact, including the reference's known
  answers (test/test_sampling.py:11-59).
* Filters: the kept set equals the oracle's (the reference's literal top-k /
  top-p code) except for tokens on the top-p boundary, |mass before - top_p|
  < 1e-5, where fp32 rounding decides; the kept probabilities agree to 2e-6
  absolute (the kernel sums exp(x - max) in 2^-40 fixed point).
* Draw: the same token as the oracle's restatement of the kernel's rule
  (Philox4x32-10 + inverse CDF) except within 1e-6 of a CDF step; and a
  chi-square test of 8192 draws against the kept distribution.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sampling_ref as S
from rwkv_tl_amd import sample_logits
from rwkv_tl_amd.sampling import Sampler, sample_into, seen_bitmap, workspace_for

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _distinct_logits(V: int, seed: int, dtype=torch.float16) -> torch.Tensor:
    """V distinct fp16 values in (-8, 8), shuffled, so no threshold falls on a tie."""
    g = torch.Generator().manual_seed(seed)
    pos = torch.arange(0, 0x4800, dtype=torch.int32)  # +0 .. just below 8
    bits = torch.cat([pos, pos[1:] | 0x8000])  # and their negatives (no -0)
    bits = bits[torch.randperm(bits.numel(), generator=g)[:V]]
    return bits.to(torch.int16).view(torch.float16).to(dtype)


def _run(logits: torch.Tensor, seed=7, offset=0, seen=None, **kw):
    kw = {"top_k": 0, "top_p": 1.0, "repetition_penalty": 1.0, **kw}
    x = logits.to(DEV).reshape(-1, logits.shape[-1])
    B, V = x.shape
    out = torch.empty(B, dtype=torch.int64, device=DEV)
    probs = torch.empty(B, V, dtype=torch.float32, device=DEV)
    sample_into(x, out, seed=seed, offset=offset, seen=seen, probs=probs, **kw)
    return out.cpu(), probs.cpu().double().numpy()


def _before_mass(l_topk: torch.Tensor) -> np.ndarray:
    """Probability mass strictly above each token among the top-k-kept logits."""
    p = torch.softmax(l_topk.double(), -1).numpy()
    order = np.argsort(-p, kind="stable")
    before = np.empty_like(p)
    before[order] = np.cumsum(p[order]) - p[order]
    return before


# ---- known answers (test/test_sampling.py:11-59) through the kernel --------------


def test_known_answers_on_gpu():
    logits = torch.tensor([1.0, 2.0, 0.5, 3.0], device=DEV)
    for t in (None, 0.0, -1.0):
        assert sample_logits(logits, temperature=t).item() == 3
    torch.manual_seed(0)
    x = torch.randn(100, device=DEV)
    for _ in range(20):
        assert sample_logits(x, temperature=1.0, top_k=1).item() == int(x.argmax())
    pair = torch.tensor([0.5, 0.4], device=DEV)
    assert sample_logits(pair, temperature=1.0, top_k=1).item() == 0
    assert sample_logits(pair, temperature=1.0, top_k=1, repetition_penalty=2.0, seen=torch.tensor([0])).item() == 1
    for _ in range(20):
        assert 0 <= sample_logits(x, temperature=1.0, top_k=50, top_p=0.9).item() < 100
    for t in (None, 0.0, 1.0):
        r = sample_logits(torch.randn(65536, device=DEV), temperature=t)
        assert r.ndim == 0 and 0 <= int(r) < 65536
    assert sample_logits(torch.randn(3, 10, device=DEV), temperature=1.0, top_p=0.5).shape == (3,)


# ---- greedy and penalty: exact -----------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("V", [65536, 50277, 1000, 13])
def test_greedy_matches_argmax(dtype, V):
    g = torch.Generator().manual_seed(V)
    logits = (torch.randn(5, V, generator=g) * 3).to(dtype)
    logits[1, V // 3] = logits[1, V // 2] = 50.0  # tie: the first index wins
    seen = torch.randint(0, V, (V // 7 + 1,), generator=g)
    for pen, sn in ((1.0, None), (1.7, seen)):
        got = sample_logits(logits.to(DEV), repetition_penalty=pen, seen=sn).cpu()
        want = S.sample_logits_ref(logits, repetition_penalty=pen, seen=sn)
        assert torch.equal(got, want)


def test_seen_bitmap_update_and_penalty():
    V = 65536
    logits = torch.zeros(2, V, dtype=torch.float16, device=DEV)
    logits[:, 123] = 5.0
    logits[:, 77] = 4.0
    logits[1, 40000] = 6.0
    smp = Sampler(V, DEV, batch=2, repetition_penalty=2.0)
    out = torch.empty(2, dtype=torch.int64, device=DEV)
    smp(logits, out)  # greedy: 123 and 40000, both marked seen
    assert out.tolist() == [123, 40000]
    bits = smp.seen.cpu()
    assert int(bits[0, 123 // 32]) & (1 << (123 % 32)) and int(bits[1, 40000 // 32]) & (1 << (40000 % 32))
    assert int(bits.ne(0).sum()) == 2
    smp(logits, out)  # 123 -> 2.5 < 4.0; 40000 -> 3.0 < 5.0
    assert out.tolist() == [77, 123]
    want = seen_bitmap(torch.tensor([123, 77]), 1, V, DEV)
    assert torch.equal(smp.seen[0:1], want)


# ---- filters and kept distribution ----------------------------------------------------

CASES = [
    dict(temperature=1.0, top_k=0, top_p=1.0),
    dict(temperature=1.0, top_k=50, top_p=1.0),
    dict(temperature=0.8, top_k=0, top_p=0.9),
    dict(temperature=0.05, top_k=0, top_p=0.9),
    dict(temperature=1.2, top_k=1000, top_p=0.5),
    dict(temperature=0.5, top_k=20, top_p=0.95),
    dict(temperature=3.0, top_k=0, top_p=0.3),
    dict(temperature=1.0, top_k=30000, top_p=0.999),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_filters_and_draw_match_oracle(case, dtype):
    kw = CASES[case]
    V = 32768
    logits = _distinct_logits(V, seed=case).to(dtype)
    pen = 1.3 if case % 2 else 1.0
    seen = torch.randperm(V, generator=torch.Generator().manual_seed(99))[:500] if pen != 1.0 else None
    bits = seen_bitmap(seen, 1, V, DEV) if seen is not None else None
    ref_l = S.filtered_logits_ref(logits, repetition_penalty=pen, seen=seen, **kw)
    want_kept = torch.isfinite(ref_l).numpy()
    want_p = S.kept_probs(ref_l)
    for offset in range(6):
        tok, p = _run(logits, seed=2024 + case, offset=offset, seen=bits, repetition_penalty=pen, **kw)
        p = p[0]
        kept = p > 0
        diff = np.nonzero(kept != want_kept)[0]
        if diff.size:
            assert kw["top_p"] < 1.0, f"kept sets differ at {diff[:8]}"
            lk = S.filtered_logits_ref(logits, repetition_penalty=pen, seen=seen, **{**kw, "top_p": 1.0})
            before = _before_mass(lk)
            assert np.all(np.abs(before[diff] - kw["top_p"]) < 1e-5), before[diff]
        np.testing.assert_allclose(p, want_p, atol=2e-6, rtol=0)
        want_tok, t, cdf = S.draw_ref(want_p, 2024 + case, offset)
        if int(tok[0]) != want_tok:
            # only where t sits on a step of the CDF, within rounding
            assert min(abs(t - cdf[want_tok]), abs(t - (cdf[want_tok - 1] if want_tok else 0.0))) < 1e-6
        assert kept[int(tok[0])]


def test_filters_with_ties_keep_whole_tie_groups():
    """fp16 logits of a 65536 vocabulary tie often. Where the reference's
    sort order splits a tie group at the top-p cutoff, the kernel keeps the
    whole group; every other token is decided the same way (up to top-p
    boundary rounding, as above)."""
    g = torch.Generator().manual_seed(5)
    logits = (torch.randn(65536, generator=g) * 2).half()
    x = logits.float().numpy()
    for kw in (dict(temperature=1.0, top_k=100), dict(temperature=0.9, top_p=0.8),
               dict(temperature=1.0, top_k=5000, top_p=0.7)):
        ref_l = S.filtered_logits_ref(logits, **kw)
        want = torch.isfinite(ref_l).numpy()
        _, p = _run(logits, **kw)
        kept = p[0] > 0
        cut = x[kept].min()
        assert np.all(kept[x > cut]) and not np.any(kept[x < cut])
        diff = np.nonzero(kept != want)[0]
        if diff.size:
            assert kw.get("top_p", 1.0) < 1.0
            lk = S.filtered_logits_ref(logits, **{**kw, "top_p": 1.0})
            before = _before_mass(lk)
            ok = (x[diff] == cut) | (np.abs(before[diff] - kw["top_p"]) < 1e-5)
            assert np.all(ok), diff[~ok][:8]


def test_threshold_bin_larger_than_the_lds_copy():
    """Two far outliers stretch the first pass's 256 equal-width bins so that
    one bin holds ~20k logits: more than the 4096 the kernel copies to LDS,
    so the thresholds are narrowed from the registers instead. (The high
    outlier stays within exp(-20) of the cluster, so no kept token's weight
    rounds to zero and "kept" can be read off the probabilities.)"""
    g = torch.Generator().manual_seed(11)
    x = torch.rand(65536, generator=g) * 0.5
    x[100], x[200] = 20.0, -60.0
    logits = x.half()
    xf = logits.float().numpy()
    for kw in (dict(temperature=1.0, top_k=1000), dict(temperature=1.0, top_p=0.5),
               dict(temperature=1.0, top_k=20000, top_p=0.9)):
        # without the high outlier (which would take all the mass) for top-p
        lg = logits.clone()
        if "top_p" in kw:
            lg[100] = 0.25
        xv = lg.float().numpy()
        ref_l = S.filtered_logits_ref(lg, **kw)
        want = torch.isfinite(ref_l).numpy()
        _, p = _run(lg, **kw)
        kept = p[0] > 0
        cut = xv[kept].min()
        assert np.all(kept[xv > cut]) and not np.any(kept[xv < cut])
        diff = np.nonzero(kept != want)[0]
        if diff.size:
            assert kw.get("top_p", 1.0) < 1.0
            before = _before_mass(S.filtered_logits_ref(lg, **{**kw, "top_p": 1.0}))
            ok = (xv[diff] == cut) | (np.abs(before[diff] - kw["top_p"]) < 1e-5)
            assert np.all(ok), diff[~ok][:8]
    assert xf[100] == 20.0


def test_draw_distribution_chi_square():
    V, B = 24, 8192
    logits = torch.linspace(-2, 2, V)
    kw = dict(temperature=0.9, top_k=18, top_p=0.95)
    p_ref = S.kept_probs(S.filtered_logits_ref(logits, **kw))
    tok, _ = _run(logits.expand(B, V).contiguous(), seed=31337, **kw)
    counts = np.bincount(tok.numpy(), minlength=V)
    keep = p_ref > 0
    assert counts[~keep].sum() == 0
    e = p_ref[keep] * B
    chi2 = float(((counts[keep] - e) ** 2 / e).sum())
    assert chi2 < 45.0, chi2  # df <= 17: p < 1e-4 under the null


def test_rows_use_distinct_streams_and_offsets_advance():
    V = 1000
    logits = torch.zeros(4, V)
    a, _ = _run(logits, seed=1, offset=0, temperature=1.0, top_k=0, top_p=1.0)
    b, _ = _run(logits, seed=1, offset=1, temperature=1.0, top_k=0, top_p=1.0)
    c, _ = _run(logits, seed=1, offset=0, temperature=1.0, top_k=0, top_p=1.0)
    assert torch.equal(a, c)
    assert len(set(a.tolist())) > 1 and not torch.equal(a, b)
    for r in range(4):
        assert int(a[r]) == S.draw_ref(np.full(V, 1.0 / V), 1, 0, r)[0]


def test_rejects_bad_arguments():
    x = torch.randn(2, 70000, device=DEV)
    with pytest.raises(ValueError):
        sample_logits(x)
    out = torch.empty(3, dtype=torch.int64, device=DEV)
    with pytest.raises(ValueError):
        sample_into(torch.randn(2, 10, device=DEV), out, temperature=1.0, top_k=0, top_p=1.0,
                    repetition_penalty=1.0, seed=0, offset=0)


# ---- the many-workgroup top-k path: the same tokens ----------------------------------


def _both_paths(logits, B, V, seen=None, offset=0, **kw):
    """The same call with and without a workspace; returns both token
    vectors and the slice counts the candidate kernel left in the workspace."""
    kw = {"top_p": 1.0, "repetition_penalty": 1.0, **kw}
    ws = workspace_for(B, V, DEV)
    outs = []
    for w in (ws, None):
        out = torch.empty(B, dtype=torch.int64, device=DEV)
        sample_into(logits, out, seed=11, offset=offset, seen=seen, workspace=w, **kw)
        outs.append(out.cpu())
    counts = ws[: B * ((V + 2047) // 2048) * 4].view(torch.int32).cpu()
    return outs[0], outs[1], counts


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("V", [65536, 50277])
def test_candidate_path_draws_the_same_tokens(dtype, V):
    """Top-k sampling with a workspace (one workgroup per 2048 logits keeps
    its slice's top-k candidates, a second launch draws from them) picks
    exactly the token the one-workgroup kernel picks, for every row, offset,
    filter setting and repetition penalty; the slice counts show the
    candidate path ran (each at least top_k and at most 128, or -1 where a
    tie group at the slice's threshold overflowed and the row went to the
    one-workgroup code)."""
    g = torch.Generator().manual_seed(V)
    B = 16
    logits = (torch.randn(B, V, generator=g) * 2).to(dtype).to(DEV)
    seen = seen_bitmap(torch.randint(0, V, (3000,), generator=g), B, V, DEV)
    for kw in (dict(temperature=1.0, top_k=50, top_p=0.9), dict(temperature=0.7, top_k=1),
               dict(temperature=1.3, top_k=128, top_p=0.5), dict(temperature=1.0, top_k=7, repetition_penalty=1.5)):
        for off in range(3):
            sn = seen if kw.get("repetition_penalty", 1.0) != 1.0 else None
            a, b, counts = _both_paths(logits, B, V, seen=sn, offset=off, **kw)
            assert torch.equal(a, b), (kw, off, a.tolist(), b.tolist())
            ok = (counts == -1) | ((counts >= kw["top_k"]) & (counts <= 128))
            assert bool(ok.all()), counts.tolist()
            if kw["top_k"] <= 50:  # (at 128, bf16's coarse values often tie past 128)
                assert float((counts > 0).float().mean()) > 0.5, counts.tolist()


def test_candidate_path_falls_back_on_a_tie_group():
    """A slice whose top-k threshold falls in a tie group of more than 128
    values (here: a constant stretch of the row) marks its count -1 and the
    row is drawn by the one-workgroup code: still the same token."""
    B, V = 4, 65536
    g = torch.Generator().manual_seed(1)
    logits = (torch.randn(B, V, generator=g) * 0.1).half()
    logits[:, 4096:8192] = 3.0  # two whole slices tied at the top
    logits = logits.to(DEV)
    for off in range(4):
        a, b, counts = _both_paths(logits, B, V, offset=off, temperature=1.0, top_k=50, top_p=0.9)
        assert torch.equal(a, b)
        assert int((counts == -1).sum()) >= B
        assert all(4096 <= int(t) < 8192 for t in a)


def test_sampler_with_workspace_updates_seen_like_without():
    B, V = 3, 65536
    logits = (torch.randn(B, V, generator=torch.Generator().manual_seed(2)) * 2).half().to(DEV)
    runs = []
    for use_ws in (True, False):
        smp = Sampler(V, DEV, batch=B, temperature=1.0, top_k=20, top_p=0.95, repetition_penalty=1.2, seed=5)
        if not use_ws:
            smp.workspace = None
        out = torch.empty(B, dtype=torch.int64, device=DEV)
        toks = []
        for _ in range(6):
            smp(logits, out)
            toks.append(out.cpu().clone())
        runs.append((torch.stack(toks), smp.seen.cpu()))
    assert torch.equal(runs[0][0], runs[1][0]) and torch.equal(runs[0][1], runs[1][1])
