"""CPU oracle: a restatement of rwkv-tl's pure-torch RWKV7 path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or the timed CPU baseline). The HIP product never calls it.

What it restates (reference citations are ``path:line`` in yuyi2439/rwkv-tl):

* ``Weights``        -- ``src/rwkv_tl/weight.py:6-184`` (transposes to
  ``[in, out]``, stacked ``rkvWt``, LN0 applied to ``emb`` at load in the
  target dtype).
* ``new_state``      -- ``src/rwkv_tl/state.py:20-44`` (per layer
  ``tmix {"x": [C] D, "rnn": [H,N,N] fp32}``, ``cmix {"x": [C] D}``), plus an
  optional leading batch dimension the reference does not have.
* ``wkv7_step``      -- ``demo/rwkv7_torch.py:49-64`` (``_dplr_rwkv``).
* ``wkv7_scan_grads`` -- gradients of the serial scan by torch autograd (the
  backward the reference plans in ``TODO.md:46-54`` has no code there).
* ``time_mix``       -- ``demo/rwkv7_torch.py:67-120``.
* ``channel_mix``    -- ``demo/rwkv7_torch.py:123-128``.
* ``decode``         -- ``demo/rwkv7_torch.py:150-158,173-178``;
  ``decode_rows`` the same for every row of a batched state at once (a speed
  path for fp32 weights, pinned to ``decode`` row by row).
* ``tmix_seq`` / ``cmix_seq`` / ``prefill`` -- ``demo/rwkv7_torch.py:160-171,
  180-257`` (serial DPLR over t, ``:227-232``).
* ``forward``        -- ``demo/_rwkv7_abc.py:74-89``.
* operator level (the CPU branches of the reference's kernel wrappers, in
  fp32): ``w_gate`` / ``v_gate`` / ``a_kk_k`` -- ``src/rwkv_tl/kernels/
  gates.py:287-313``; ``gates`` -- ``gates.py:315-357``; ``rank_gemv`` --
  ``gates.py:254-285``; ``l2norm_neg_kk_a`` -- ``src/rwkv_tl/kernels/
  dplr.py:229-235``; ``gn_rkrk`` -- ``dplr.py:237-254``. They are pinned by
  composing them into one token of ``time_mix`` (golden-pinned) and by the
  closed forms of each formula (tests/test_oracle.py).

The op order and dtypes of every torch call follow the reference line by line,
so that with fp16 weights it reproduces the reference's fp16 rounding points
and with fp32 weights it is the exact-fp32 model. A batched state (leading B)
is handled by running each row as its own single-sequence state, which is the
reference's semantics for one sequence.

``wkv7_brute`` is an independent pure-Python loop version of the DPLR step
(no einsum, no torch) used to pin ``wkv7_step`` on tiny inputs.

Parity pins for this module (tests/test_oracle.py): golden vectors written by
the reference's own pure-torch path (tests/golden/), closed forms of the DPLR
update, F.layer_norm / F.group_norm library routines, and brute-force loops.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import Tensor

N_HEAD_DIM = 64
GN_EPS = 64e-5  # demo/rwkv7_torch.py:114
SQRT_E = math.e**0.5  # demo/rwkv7_torch.py:103 (torch.e ** 0.5)


# --------------------------------------------------------------------------
# Weights (src/rwkv_tl/weight.py)
# --------------------------------------------------------------------------


class _LN:
    """LayerNorm weights; ``weight.py:6-15`` (F.layer_norm, default eps 1e-5)."""

    def __init__(self, sd: dict[str, Tensor], prefix: str) -> None:
        self.w = sd[f"{prefix}.weight"]
        self.b = sd[f"{prefix}.bias"]

    def __call__(self, x: Tensor) -> Tensor:
        return F.layer_norm(x, (x.shape[-1],), self.w, self.b)


class _Att:
    """Attention weights; ``weight.py:66-106``."""

    def __init__(self, sd: dict[str, Tensor], p: str, ln_pre: _LN) -> None:
        self.ln_pre = ln_pre
        self.ln_x = _LN(sd, f"{p}.ln_x")
        for name in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"):
            setattr(self, name, sd[f"{p}.{name}"].squeeze())
        for name in ("w0", "w1", "w2", "a0", "a1", "a2", "v0", "v1", "v2", "g1", "g2"):
            setattr(self, name, sd[f"{p}.{name}"])
        self.g1t = sd[f"{p}.g1"].t().contiguous()
        self.r_k = sd[f"{p}.r_k"]
        self.k_k = sd[f"{p}.k_k"]
        self.k_a = sd[f"{p}.k_a"]
        # Checkpoint matrices are [out, in]; the reference keeps [in, out].
        self.rkvWt = torch.stack(
            [sd[f"{p}.{m}.weight"].T.contiguous() for m in ("receptance", "key", "value")]
        )
        self.oWt = sd[f"{p}.output.weight"].T.contiguous()


class _Ffn:
    """FFN weights; ``weight.py:122-126``."""

    def __init__(self, sd: dict[str, Tensor], p: str, ln_pre: _LN) -> None:
        self.ln_pre = ln_pre
        self.x_k = sd[f"{p}.x_k"].squeeze()
        self.kWt = sd[f"{p}.key.weight"].T.contiguous()
        self.vWt = sd[f"{p}.value.weight"].T.contiguous()


class _Block:
    def __init__(self, sd: dict[str, Tensor], p: str) -> None:
        self.att = _Att(sd, f"{p}.att", _LN(sd, f"{p}.ln1"))
        self.ffn = _Ffn(sd, f"{p}.ffn", _LN(sd, f"{p}.ln2"))


class Weights:
    """Restatement of ``RWKV7Weight`` (``weight.py:155-184``) from a state dict.

    ``dtype`` is applied to every tensor first (``weight.py:167-169``); then
    the embedding is layer-normalised once with ``blocks.0.ln0`` in that dtype
    (``weight.py:175``).
    """

    def __init__(
        self,
        sd: dict[str, Tensor],
        dtype: torch.dtype = torch.float32,
        device: str | torch.device = "cpu",
    ) -> None:
        sd = {k: v.to(device=device, dtype=dtype) for k, v in sd.items()}
        self.dtype = dtype
        self.head = sd["head.weight"]
        self.ln_out = _LN(sd, "ln_out")
        self.emb = _LN(sd, "blocks.0.ln0")(sd["emb.weight"])
        self.L = 1 + max(int(k.split(".")[1]) for k in sd if k.startswith("blocks."))
        self.C = self.emb.shape[1]
        self.H = self.C // N_HEAD_DIM
        self.blocks = [_Block(sd, f"blocks.{i}") for i in range(self.L)]

    @classmethod
    def from_emb(cls, sd: dict[str, Tensor], emb: Tensor, dtype: torch.dtype) -> "Weights":
        """Like ``__init__`` but take an already LN0'd embedding table as is.

        Used when the device under test computed LN0 itself, so that both sides
        start from bit-identical embedding rows.
        """
        w = cls(sd, dtype=dtype)
        w.emb = emb.to(device="cpu", dtype=dtype)
        return w


# --------------------------------------------------------------------------
# State (src/rwkv_tl/state.py)
# --------------------------------------------------------------------------


def new_state(
    L: int,
    C: int,
    N: int = N_HEAD_DIM,
    *,
    dtype: torch.dtype = torch.float16,
    batch: int | None = None,
    device: str | torch.device = "cpu",
) -> tuple[list[dict[str, Tensor]], list[dict[str, Tensor]]]:
    """Zero state, ``state.py:20-44``; ``batch`` adds a leading dimension."""
    lead = () if batch is None else (batch,)
    H = C // N
    tmix = [
        {
            "x": torch.zeros(lead + (C,), dtype=dtype, device=device),
            "rnn": torch.zeros(lead + (H, N, N), dtype=torch.float32, device=device),
        }
        for _ in range(L)
    ]
    cmix = [{"x": torch.zeros(lead + (C,), dtype=dtype, device=device)} for _ in range(L)]
    return tmix, cmix


def _row(state, b: int):
    """Views of batch row ``b`` of a batched state (shares storage)."""
    tmix, cmix = state
    return (
        [{k: v[b] for k, v in d.items()} for d in tmix],
        [{k: v[b] for k, v in d.items()} for d in cmix],
    )


# --------------------------------------------------------------------------
# Math helpers (demo/rwkv7_torch.py:26-64)
# --------------------------------------------------------------------------


def _lerp(x: Tensor, y: Tensor, w: Tensor) -> Tensor:
    # demo/rwkv7_torch.py:34-35
    return x + w * (y - x)


def _l2_normalize(x: Tensor) -> Tensor:
    # demo/rwkv7_torch.py:38-41
    den = torch.sqrt(torch.sum(x * x, dim=-1, keepdim=True))
    return x / torch.clamp(den, min=1e-12)


def wkv7_step(S: Tensor, r, w, k, v, a, b) -> tuple[Tensor, Tensor]:
    """One DPLR step for all heads; ``demo/rwkv7_torch.py:49-64``.

    ``S[h, v, k]`` (value row, key column), fp32. ``a`` is the normalised key
    the state is projected on, ``b`` the rank-1 write direction:
    ``S' = S diag(w) + (S a) b^T + v k^T``, ``y = S' r`` cast to ``v.dtype``.
    """
    S_new = (
        torch.einsum("hvk,hk->hvk", S, w.float())
        + torch.einsum("hva,ha,hb->hvb", S, a.float(), b.float())
        + torch.einsum("hv,hk->hvk", v.float(), k.float())
    )
    y = torch.einsum("hvk,hk->hv", S_new, r.float())
    return y.to(v.dtype), S_new


def wkv7_scan(S: Tensor, r, w, k, v, a, b) -> tuple[Tensor, Tensor]:
    """Serial DPLR over a batch of sequences.

    Inputs ``r, w, k, v, a, b`` are ``[B, T, H, N]``; ``S`` is ``[B, H, N, N]``
    fp32 and is left untouched. Returns ``(y [B,T,H,N] in v.dtype, S_T)``.
    Follows the per-token loop of ``demo/rwkv7_torch.py:227-232`` for each
    sequence.
    """
    Bsz, T = r.shape[:2]
    S = S.clone().float()
    y = torch.empty(r.shape, dtype=v.dtype, device=r.device)
    for bi in range(Bsz):
        for t in range(T):
            y[bi, t], S[bi] = wkv7_step(
                S[bi], r[bi, t], w[bi, t], k[bi, t], v[bi, t], a[bi, t], b[bi, t]
            )
    return y, S


def wkv7_scan_grads(S: Tensor, r, w, k, v, a, b, gy: Tensor, gS: Tensor | None = None):
    """Gradients of ``wkv7_scan`` (fp32) by torch autograd: of
    ``L = <gy, y> + <gS, S_T>`` with respect to ``(S, r, w, k, v, a, b)``.

    The reference has no backward (``TODO.md:46-54`` plans one); the gradient
    is fixed by the forward restated above, so the checker differentiates that
    forward with autograd. Pinned in tests/test_oracle.py by finite differences
    of ``wkv7_brute`` (double precision, no torch)."""
    xs = [t.detach().float().clone().requires_grad_(True) for t in (S, r, w, k, v, a, b)]
    with torch.enable_grad():
        # the per-token loop of wkv7_scan without its in-place stores
        ys, finals = [], []
        for bi in range(r.shape[0]):
            St, yb = xs[0][bi], []
            for t in range(r.shape[1]):
                yt, St = wkv7_step(St, *(x[bi, t] for x in xs[1:]))
                yb.append(yt)
            ys.append(torch.stack(yb))
            finals.append(St)
        y, S_T = torch.stack(ys), torch.stack(finals)
        L = (y.float() * gy.float()).sum()
        if gS is not None:
            L = L + (S_T * gS.float()).sum()
        return torch.autograd.grad(L, xs)


def wkv7_brute(S, r, w, k, v, a, b):
    """Pure-Python loops over nested lists; independent of torch and einsum.

    ``S`` is ``[H][N][N]``; vectors are ``[T][H][N]``. Returns ``(y, S)`` as
    lists of Python floats (double precision).
    """
    H = len(S)
    N = len(S[0])
    S = [[list(row) for row in head] for head in S]
    ys = []
    for t in range(len(r)):
        yt = []
        for h in range(H):
            Sh = S[h]
            sa = [sum(Sh[i][j] * a[t][h][j] for j in range(N)) for i in range(N)]
            for i in range(N):
                for j in range(N):
                    Sh[i][j] = Sh[i][j] * w[t][h][j] + sa[i] * b[t][h][j] + v[t][h][i] * k[t][h][j]
            yt.append([sum(Sh[i][j] * r[t][h][j] for j in range(N)) for i in range(N)])
        ys.append(yt)
    return ys, S


# --------------------------------------------------------------------------
# One token (demo/rwkv7_torch.py:67-128)
# --------------------------------------------------------------------------


def time_mix(att: _Att, x0: Tensor, v_first, st: dict[str, Tensor], H: int, N: int):
    """``demo/rwkv7_torch.py:67-120`` for one token of one sequence."""
    x = att.ln_pre(x0)
    prev = st["x"]
    xr = _lerp(x, prev, att.x_r)
    xw = _lerp(x, prev, att.x_w)
    xk = _lerp(x, prev, att.x_k)
    xv = _lerp(x, prev, att.x_v)
    xa = _lerp(x, prev, att.x_a)
    xg = _lerp(x, prev, att.x_g)
    st["x"].copy_(x)  # after every read of prev (:84-86)

    r = xr @ att.rkvWt[0]
    k = xk @ att.rkvWt[1]
    v = xv @ att.rkvWt[2]
    if v_first is None:
        v_first = v
    else:
        v = _lerp(v, v_first, torch.sigmoid(att.v0.reshape(-1) + xv @ att.v1 @ att.v2))
    w = torch.exp(-torch.sigmoid(att.w0.reshape(-1) + torch.tanh(xw @ att.w1) @ att.w2) / SQRT_E)
    a = torch.sigmoid(att.a0.reshape(-1) + xa @ att.a1 @ att.a2)
    kk = k * att.k_k.reshape(-1)
    k = _lerp(k, k * a, att.k_a.reshape(-1))

    r, w, k, v, kk, a = [z.reshape(H, N) for z in (r, w, k, v, kk, a)]
    kk = _l2_normalize(kk)
    y, S_new = wkv7_step(st["rnn"], r, w, k, v, kk, -kk * a)
    st["rnn"].copy_(S_new)
    y = F.group_norm(y.reshape(1, H * N), H, att.ln_x.w, att.ln_x.b, GN_EPS).reshape(-1)
    y += (torch.sum(r * k * att.r_k, dim=1, keepdim=True) * v).reshape(-1)
    g = torch.mv(att.g2.T.contiguous(), torch.sigmoid(torch.mv(att.g1t, xg)))
    return torch.add(x0, (y * g) @ att.oWt), v_first


def channel_mix(ffn: _Ffn, x0: Tensor, st: dict[str, Tensor]) -> Tensor:
    """``demo/rwkv7_torch.py:123-128``."""
    x_ln = ffn.ln_pre(x0)
    x = _lerp(x_ln, st["x"], ffn.x_k)
    st["x"].copy_(x_ln)
    return torch.add(x0, F.relu(x @ ffn.kWt) ** 2 @ ffn.vWt)


def _decode_one(W: Weights, token: Tensor, state) -> Tensor:
    # demo/rwkv7_torch.py:150-158 with EMB :173-175 and HEAD :177-178
    x = F.embedding(token, W.emb)
    x = x.squeeze(0) if x.dim() > 1 else x
    v_first = None
    tmix, cmix = state
    for i, blk in enumerate(W.blocks):
        x, v_first = time_mix(blk.att, x, v_first, tmix[i], W.H, N_HEAD_DIM)
        x = channel_mix(blk.ffn, x, cmix[i])
    return torch.mv(W.head, W.ln_out(x))


def decode(W: Weights, token: Tensor, state):
    """One decode step. ``token`` is 0-d / ``[1]`` (single state) or ``[B]``.

    Returns ``(logits, state)``: ``[V]`` for a single state, ``[B, V]`` for a
    batched one (row ``b`` = a single-sequence decode of state row ``b``).
    """
    batched = state[0][0]["rnn"].dim() == 4
    if not batched:
        return _decode_one(W, token.reshape(-1)[:1] if token.dim() else token, state), state
    rows = [
        _decode_one(W, token.reshape(-1)[b : b + 1], _row(state, b))
        for b in range(state[0][0]["rnn"].shape[0])
    ]
    return torch.stack(rows), state


def _time_mix_rows(att: _Att, x0: Tensor, v_first, st: dict[str, Tensor], H: int, N: int):
    """``time_mix`` for one token of each of B sequences at once (x0 [B, C],
    state rows [B, ...]): the same formulas with every matrix product taken
    for all rows together. A speed path of the checker for fp32 weights;
    pinned to ``time_mix`` row by row in tests/test_oracle.py."""
    B = x0.shape[0]
    x = att.ln_pre(x0)
    prev = st["x"]
    xr = _lerp(x, prev, att.x_r)
    xw = _lerp(x, prev, att.x_w)
    xk = _lerp(x, prev, att.x_k)
    xv = _lerp(x, prev, att.x_v)
    xa = _lerp(x, prev, att.x_a)
    xg = _lerp(x, prev, att.x_g)
    st["x"].copy_(x)
    r = xr @ att.rkvWt[0]
    k = xk @ att.rkvWt[1]
    v = xv @ att.rkvWt[2]
    if v_first is None:
        v_first = v
    else:
        v = _lerp(v, v_first, torch.sigmoid(att.v0.reshape(-1) + xv @ att.v1 @ att.v2))
    w = torch.exp(-torch.sigmoid(att.w0.reshape(-1) + torch.tanh(xw @ att.w1) @ att.w2) / SQRT_E)
    a = torch.sigmoid(att.a0.reshape(-1) + xa @ att.a1 @ att.a2)
    kk = k * att.k_k.reshape(-1)
    k = _lerp(k, k * a, att.k_a.reshape(-1))
    r, w, k, v, kk, a = [z.reshape(B, H, N) for z in (r, w, k, v, kk, a)]
    kk = _l2_normalize(kk)
    S = st["rnn"]
    b = -kk * a
    S_new = (
        torch.einsum("zhvk,zhk->zhvk", S, w.float())
        + torch.einsum("zhva,zha,zhb->zhvb", S, kk.float(), b.float())
        + torch.einsum("zhv,zhk->zhvk", v.float(), k.float())
    )
    y = torch.einsum("zhvk,zhk->zhv", S_new, r.float()).to(v.dtype)
    st["rnn"].copy_(S_new)
    y = F.group_norm(y.reshape(B, H * N), H, att.ln_x.w, att.ln_x.b, GN_EPS)
    y = y + (torch.sum(r * k * att.r_k, dim=-1, keepdim=True) * v).reshape(B, -1)
    g = torch.sigmoid(xg @ att.g1) @ att.g2
    return x0 + (y * g) @ att.oWt, v_first.reshape(B, -1)


def _channel_mix_rows(ffn: _Ffn, x0: Tensor, st: dict[str, Tensor]) -> Tensor:
    """``channel_mix`` for B rows at once (see ``_time_mix_rows``)."""
    x_ln = ffn.ln_pre(x0)
    x = _lerp(x_ln, st["x"], ffn.x_k)
    st["x"].copy_(x_ln)
    return x0 + F.relu(x @ ffn.kWt) ** 2 @ ffn.vWt


def decode_rows(W: Weights, token: Tensor, state):
    """``decode`` of a batched state (token [B]) with every row computed in
    the same batched torch operations instead of one row at a time: the same
    model, ~B times fewer passes over the weights. For fp32 weights (the
    fp32-math oracle) only; rows agree with ``decode`` to fp32 rounding
    (tests/test_oracle.py). Returns ``(logits [B, V], state)``."""
    tmix, cmix = state
    x = F.embedding(token.reshape(-1), W.emb)
    v_first = None
    for i, blk in enumerate(W.blocks):
        x, v_first = _time_mix_rows(blk.att, x, v_first, tmix[i], W.H, N_HEAD_DIM)
        x = _channel_mix_rows(blk.ffn, x, cmix[i])
    return W.ln_out(x) @ W.head.T, state


# --------------------------------------------------------------------------
# Sequence (demo/rwkv7_torch.py:160-171,180-257)
# --------------------------------------------------------------------------


def tmix_seq(att: _Att, x0: Tensor, v_first, st, H: int, N: int):
    """``demo/rwkv7_torch.py:185-242``: batched over T, DPLR serial in t."""
    T_len = x0.shape[0]
    x = att.ln_pre(x0)
    prev = torch.cat([st["x"].unsqueeze(0), x[:-1]], dim=0)
    xr = _lerp(x, prev, att.x_r)
    xw = _lerp(x, prev, att.x_w)
    xk = _lerp(x, prev, att.x_k)
    xv = _lerp(x, prev, att.x_v)
    xa = _lerp(x, prev, att.x_a)
    xg = _lerp(x, prev, att.x_g)
    st["x"].copy_(x[-1])

    r, k, v = torch.bmm(torch.stack([xr, xk, xv], 0), att.rkvWt).unbind(0)
    if v_first is None:
        v_first = v
    else:
        v = _lerp(v, v_first, torch.sigmoid(att.v0.reshape(-1) + xv @ att.v1 @ att.v2))
    w = torch.exp(-torch.sigmoid(att.w0.reshape(-1) + torch.tanh(xw @ att.w1) @ att.w2) / SQRT_E)
    a = torch.sigmoid(att.a0.reshape(-1) + xa @ att.a1 @ att.a2)
    kk = k * att.k_k.reshape(-1)
    k = _lerp(k, k * a, att.k_a.reshape(-1))

    r, w, k, v, kk, a = [z.view(T_len, H, N) for z in (r, w, k, v, kk, a)]
    kk = _l2_normalize(kk)
    neg_kk_a = -kk * a
    y = torch.empty(T_len, H, N, dtype=x0.dtype, device=x0.device)
    for t in range(T_len):
        y_t, S_new = wkv7_step(st["rnn"], r[t], w[t], k[t], v[t], kk[t], neg_kk_a[t])
        st["rnn"].copy_(S_new)
        y[t] = y_t
    y = F.group_norm(y.reshape(T_len, H * N), H, att.ln_x.w, att.ln_x.b, GN_EPS)
    rkrk = torch.sum(r * k * att.r_k, dim=-1, keepdim=True)
    y = (y.view(T_len, H, N) + rkrk * v).reshape(T_len, H * N)
    g = torch.sigmoid(xg @ att.g1) @ att.g2
    return x0 + (y * g) @ att.oWt, v_first


def cmix_seq(ffn: _Ffn, x0: Tensor, st) -> Tensor:
    """``demo/rwkv7_torch.py:250-255``."""
    x_ln = ffn.ln_pre(x0)
    prev = torch.cat([st["x"].unsqueeze(0), x_ln[:-1]], dim=0)
    x = _lerp(x_ln, prev, ffn.x_k)
    st["x"].copy_(x_ln[-1])
    return x0 + F.relu(x @ ffn.kWt) ** 2 @ ffn.vWt


def _prefill_one(W: Weights, tokens: Tensor, state) -> None:
    # demo/rwkv7_torch.py:160-171
    if tokens.numel() == 0:
        raise RuntimeError("prefill received an empty token sequence")
    x = F.embedding(tokens, W.emb)
    v_first = None
    tmix, cmix = state
    for i, blk in enumerate(W.blocks):
        x, v_first = tmix_seq(blk.att, x, v_first, tmix[i], W.H, N_HEAD_DIM)
        x = cmix_seq(blk.ffn, x, cmix[i])


def prefill(W: Weights, tokens: Tensor, state):
    """Prefill ``tokens`` ``[T]`` (single state) or ``[B, T]`` (batched)."""
    batched = state[0][0]["rnn"].dim() == 4
    if not batched:
        _prefill_one(W, tokens.reshape(-1), state)
        return state
    for b in range(tokens.shape[0]):
        _prefill_one(W, tokens[b], _row(state, b))
    return state


def forward(W: Weights, tokens: Tensor, state):
    """``demo/_rwkv7_abc.py:74-89``: prefill all but the last, decode the last."""
    if tokens.dim() == 0 or tokens.numel() == 1:
        return decode(W, tokens.reshape(-1), state)
    prefill(W, tokens[:-1], state)
    return decode(W, tokens[-1:], state)


# --------------------------------------------------------------------------
# Operator level: the time-mix stages one by one (fp32 arithmetic)
# --------------------------------------------------------------------------


def _f(*ts: Tensor) -> list[Tensor]:
    return [t.float() for t in ts]


def w_gate(x: Tensor, w0: Tensor) -> Tensor:
    # src/rwkv_tl/kernels/gates.py:287-291
    x, w0 = _f(x, w0)
    return torch.exp(-torch.sigmoid(w0 + x) / SQRT_E)


def v_gate(v: Tensor, v_first: Tensor, v0: Tensor, v12: Tensor) -> Tensor:
    # gates.py:293-297
    v, v_first, v0, v12 = _f(v, v_first, v0, v12)
    return v + torch.sigmoid(v0 + v12) * (v_first - v)


def a_kk_k(a0: Tensor, a_x: Tensor, k: Tensor, k_k: Tensor, k_a: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    # gates.py:299-313
    a0, a_x, k, k_k, k_a = _f(a0, a_x, k, k_k, k_a)
    a = torch.sigmoid(a0 + a_x)
    return a, k * k_k, k + k_a * (k * a - k)


def gates(vr, wr, ar, gr, v, v_first, k, v2t, w2t, a2t, g2t, v0, w0, a0, k_k, k_a):
    """gates.py:315-357: returns ``(v, w, a, kk, k, g)``."""
    vr, wr, ar, gr, v, v_first, k, v2t, w2t, a2t, g2t, v0, w0, a0, k_k, k_a = _f(
        vr, wr, ar, gr, v, v_first, k, v2t, w2t, a2t, g2t, v0, w0, a0, k_k, k_a
    )
    v12 = v2t @ vr
    w12 = w2t @ torch.tanh(wr)
    a12 = a2t @ ar
    g12 = g2t @ torch.sigmoid(gr)
    v_out = v + torch.sigmoid(v0 + v12) * (v_first - v)
    w_out = torch.exp(-torch.sigmoid(w0 + w12) / SQRT_E)
    a = torch.sigmoid(a0 + a12)
    return v_out, w_out, a, k * k_k, k + k_a * (k * a - k), g12


def rank_gemv(xv, xw, xa, xg, packed, rv: int, rw: int, ra: int, rg: int) -> Tensor:
    # gates.py:254-285 (rows of the packed [v1t; w1t; a1t; g1t] by segment)
    xv, xw, xa, xg, packed = _f(xv, xw, xa, xg, packed)
    return torch.cat(
        [
            packed[:rv] @ xv,
            packed[rv : rv + rw] @ xw,
            packed[rv + rw : rv + rw + ra] @ xa,
            packed[rv + rw + ra : rv + rw + ra + rg] @ xg,
        ]
    )


def l2norm_neg_kk_a(kk: Tensor, a: Tensor) -> tuple[Tensor, Tensor]:
    # src/rwkv_tl/kernels/dplr.py:229-235, per head over dim 1
    kk, a = _f(kk, a)
    den = torch.sqrt(torch.sum(kk * kk, dim=1, keepdim=True))
    kn = kk / torch.clamp(den, min=1e-12)
    return kn, -kn * a


def gn_rkrk(y, r, k, v, r_k, ln_w, ln_b) -> Tensor:
    # dplr.py:237-254: GroupNorm over heads (eps 64e-5) + (sum r k r_k) v
    y, r, k, v, r_k, ln_w, ln_b = _f(y, r, k, v, r_k, ln_w, ln_b)
    h, n = y.shape
    yf = F.group_norm(y.reshape(1, h * n), h, ln_w, ln_b, GN_EPS).reshape(-1)
    return yf + (torch.sum(r * k * r_k, dim=1, keepdim=True) * v).reshape(-1)
