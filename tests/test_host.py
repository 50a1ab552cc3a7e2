"""Host-side tests (CPU only): the C ABI library, layouts, State, weights,
sampling and the model factory. No kernel is launched here."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from oracle import rwkv7_ref as R
from oracle import sampling_ref as S
from rwkv_tl_amd import _lib, make_rwkv7, sample_logits
from rwkv_tl_amd.checkpoint import SHAPES, make_random_state_dict
from rwkv_tl_amd.state import State
from rwkv_tl_amd.weight import RWKV7Weight, layer_layout, model_dims, quantize_rows_i8, to_fragments

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "rwkv7_hip.h"


def _header_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(rwkv7_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    declared = _header_functions()
    assert declared == sorted(_lib.SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.rwkv7_abi_version() == _lib.ABI_VERSION
    assert lib.rwkv7_strerror(2) == b"unsupported shape"


def _dims(shape="0.4b") -> _lib.Dims:
    s = SHAPES[shape]
    return _lib.Dims(s.n_layer, s.n_embd, s.n_head, s.n_ffn, s.vocab, s.rank_w, s.rank_a, s.rank_v, s.rank_g)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the decision on a host without a GPU")
@pytest.mark.parametrize("shape", ["tiny", "0.4b"])
def test_decode_path_decision_without_a_device(shape):
    """The persistent decode kernel is chosen only when the device's CU count
    and occupancy for it are known to fit its grid at once; with no device
    (this host) the library reports the multi-launch path: embed, six launches
    per layer and the head for batch 1; embed, seven per layer, LayerNorm and
    head GEMM for a batch. The model flag gives the same count on any host."""
    lib = _lib.load()
    d = _dims(shape)
    m = _lib.Model(dims=d)
    L = d.n_layer
    assert lib.rwkv7_decode_launches(ctypes.byref(m), 1, 1) == 1 + 6 * L + 1
    assert lib.rwkv7_decode_launches(ctypes.byref(m), 1, 0) == 1 + 6 * L
    assert lib.rwkv7_decode_launches(ctypes.byref(m), 4, 1) == 1 + 7 * L + 2
    m.flags = _lib.MODEL_MULTI_LAUNCH_DECODE
    assert lib.rwkv7_decode_launches(ctypes.byref(m), 1, 1) == 1 + 6 * L + 1
    assert lib.rwkv7_decode_launches(None, 1, 1) == -1


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the decision on a host without a GPU")
def test_f32_activation_decision_without_a_device():
    """Batched steps keep f32 activations (two 16-bit MFMA parts) unless some
    GEMM of the layer would take the large-M path: with 256 CUs that needs
    ceil(M / 128) * ceil(N / 128) >= 512 tiles, so the widest matrix (the FFN,
    N = F) sets the threshold: M >= 1921 rows at F = 4096, M >= 897 at
    F = 8192. Long prefills beyond it round the operands to 16 bits."""
    lib = _lib.load()
    f32 = lambda shape, B, T: lib.rwkv7_step_f32_activations(  # noqa: E731
        ctypes.byref(_lib.Model(dims=_dims(shape))), B, T)
    assert f32("0.4b", 1, 128) == 1
    assert f32("0.4b", 16, 16) == 1
    assert f32("0.4b", 1, 1920) == 1
    assert f32("0.4b", 1, 1921) == 0
    assert f32("0.4b", 130, 1) == 1
    assert f32("1.5b", 64, 1) == 1
    assert f32("1.5b", 2, 448) == 1
    assert f32("1.5b", 1, 897) == 0
    assert f32("1.5b", 4, 1024) == 0
    assert f32("0.4b", 0, 1) == -1
    assert lib.rwkv7_step_f32_activations(None, 1, 1) == -1


@pytest.mark.parametrize("shape", ["tiny", "0.1b", "0.4b", "1.5b"])
def test_layer_layout(shape):
    d = _dims(shape)
    lay = layer_layout(d)
    C, F = d.n_embd, d.n_ffn
    SR = d.rank_w + d.rank_a + d.rank_v + d.rank_g
    offs = [lay.w_rkv, lay.w_lora1, lay.w_lora2, lay.w_o, lay.w_fk, lay.w_fv, lay.vec, lay.bytes]
    assert offs == sorted(offs)
    assert lay.w_lora1 == lay.w_rkv + 3 * C * C * 2  # one [3C+SR, C] decode matrix
    assert lay.w_lora2 >= lay.w_lora1 + SR * C * 2
    assert lay.w_o >= lay.w_lora2 + C * SR * 2
    assert lay.w_fk >= lay.w_o + C * C * 2
    assert lay.w_fv >= lay.w_fk + F * C * 2
    assert lay.vec >= lay.w_fv + C * F * 2
    assert lay.bytes >= lay.vec + _lib.NVEC * C * 4
    assert all(o % 256 == 0 for o in offs if o != lay.w_lora1)
    # fragment arena: every matrix padded to 16 x 32 blocks, in order, no overlap
    def fb(n, k):
        return (-(-n // 16) * 16) * (-(-k // 32) * 32) * 2

    R = (d.rank_v, d.rank_w, d.rank_a, d.rank_g)
    regions = [(lay.f_rkv, fb(3 * C, C))] + [(lay.f_l1[g], fb(R[g], C)) for g in range(4)]
    regions += [(lay.f_l2[g], fb(C, R[g])) for g in range(4)]
    regions += [(lay.f_o, fb(C, C)), (lay.f_fk, fb(F, C)), (lay.f_fv, fb(C, F))]
    for (o0, n0), (o1, _) in zip(regions, regions[1:]):
        assert o0 % 256 == 0 and o1 >= o0 + n0
    assert lay.frag_bytes >= regions[-1][0] + regions[-1][1] and lay.frag_bytes % 256 == 0
    # int8 arena: q_rkv [3C+SR, C], q_o, q_fk, q_fv, then the f32 row scales
    q = [(lay.q_rkv, (3 * C + SR) * C), (lay.q_o, C * C), (lay.q_fk, F * C), (lay.q_fv, C * F),
         (lay.q_scale, 4 * (3 * C + SR + C + F + C))]
    for (o0, n0), (o1, _) in zip(q, q[1:]):
        assert o0 % 256 == 0 and o1 >= o0 + n0
    assert lay.q_bytes >= q[-1][0] + q[-1][1] and lay.q_bytes % 256 == 0
    assert _lib.load().rwkv7_head_q_scale_offset(ctypes.byref(d)) >= d.vocab * C


def test_fragment_order_matches_header_definition():
    """Block (s, j) of W [N, K] is 1024 bytes at (s * K'/32 + j) * 1024 and its
    lane l holds W[16 s + l % 16, 32 j + 8 (l // 16) : +8], zero-padded."""
    N, K = 37, 70  # both ragged: padded to 48 x 96
    W = torch.arange(N * K, dtype=torch.float32).view(N, K) + 1
    f = to_fragments(W)
    Np, Kp = 48, 96
    assert f.numel() == Np * Kp
    blocks = f.view(Np // 16, Kp // 32, 64, 8)
    for s in range(Np // 16):
        for j in range(Kp // 32):
            for lane in range(64):
                r, k0 = 16 * s + lane % 16, 32 * j + 8 * (lane // 16)
                want = torch.zeros(8)
                if r < N:
                    ks = [k for k in range(k0, k0 + 8) if k < K]
                    want[: len(ks)] = W[r, ks[0] : ks[-1] + 1] if ks else want[:0]
                assert torch.equal(blocks[s, j, lane], want), (s, j, lane)


def test_layout_rejects_unsupported_dims():
    lib = _lib.load()
    out = _lib.LayerLayout()
    bad = [
        dict(n_embd=768 + 64),   # not a multiple of 256
        dict(n_head=10),          # n_head * 64 != n_embd
        dict(rank_w=60),          # rank not a multiple of 8
        dict(n_ffn=1000),
    ]
    for change in bad:
        d = _dims("0.4b")
        for k, v in change.items():
            setattr(d, k, v)
        if "n_embd" in change:
            d.n_head = d.n_embd // 64
        assert lib.rwkv7_layer_layout_get(ctypes.byref(d), ctypes.byref(out)) == 2, change
    assert lib.rwkv7_layer_layout_get(None, ctypes.byref(out)) == 1


def test_workspace_and_entry_point_argument_errors():
    lib = _lib.load()
    d = _dims("0.4b")
    assert lib.rwkv7_workspace_bytes(ctypes.byref(d), 1, 1) > 0
    assert lib.rwkv7_workspace_bytes(ctypes.byref(d), 4, 128) > lib.rwkv7_workspace_bytes(ctypes.byref(d), 1, 1)
    assert lib.rwkv7_workspace_bytes(ctypes.byref(d), 0, 1) == -1
    # null descriptors are rejected on the host before any launch
    assert lib.rwkv7_decode(None, None, None, None, None, 0, None) == 1
    model = _lib.Model(dims=d)
    st = _lib.StateDesc(batch=1)
    assert lib.rwkv7_decode(ctypes.byref(model), ctypes.byref(st), None, None, None, 0, None) == 1
    assert lib.rwkv7_wkv7(None, None, None, 0, None, None, None, None, None, 1, 1, 1, 0, None) == 1
    assert lib.rwkv7_gemm_f16(1, 8, 1, 8, 1, 8, 1, 8, 8, 9, 0, None) == 1  # bad epilogue code
    assert lib.rwkv7_gemv_f16(1, 1, 100, 1, 4, 100, 0, None) == 2       # K % 256
    assert lib.rwkv7_gemv_i8(None, 16, 16, 16, 16, 4, 16, None) == 1  # null x
    assert lib.rwkv7_gemv_i8(16, 16, 24, 16, 16, 4, 24, None) == 2    # K % 16
    assert lib.rwkv7_gemv_i8(16, 16, 16, 16, 16, 4, 16384, None) == 2  # K > 8192
    assert lib.rwkv7_gemv_i8(16, 16, 32, 16, 16, 4, 48, None) == 2    # ldq < K
    assert lib.rwkv7_gemv_i8(16, 8, 16, 16, 16, 4, 16, None) == 2     # Q not 16-byte aligned
    assert lib.rwkv7_lerp(1, 1, 1, 3, 1, None, 8, 0, None) == 2          # n_mix not 1 or 6


def test_state_layout_and_arena():
    S = State(3, 256, 64, dtype=torch.float16)
    assert len(S.tmix) == 3 and len(S.cmix) == 3
    assert S.tmix[0]["x"].shape == (256,) and S.tmix[0]["x"].dtype == torch.float16
    assert S.tmix[0]["rnn"].shape == (4, 64, 64) and S.tmix[0]["rnn"].dtype == torch.float32
    assert S.cmix[2]["x"].shape == (256,)
    assert S.arena_intact()
    S.tmix[1]["x"].fill_(1.0)
    assert S.arenas[0][1].float().sum() == 256
    S.reset()
    assert S.arenas[0].abs().sum() == 0
    S.tmix[1]["x"] = torch.zeros(256, dtype=torch.float16)  # a rebind
    assert not S.arena_intact()
    Sb = State(2, 256, 64, batch=5)
    assert Sb.tmix[0]["rnn"].shape == (5, 4, 64, 64) and Sb.cmix[1]["x"].shape == (5, 256)
    with pytest.raises(ValueError):
        State(2, 100, 64)


def test_weight_matches_oracle_restatement():
    sd = make_random_state_dict("tiny", seed=0, dtype=torch.float32)
    w = RWKV7Weight.from_state_dict(sd, device="cpu", dtype=torch.float16)
    o = R.Weights(sd, torch.float16)
    assert (w.L, w.C) == (o.L, o.C)
    assert torch.equal(w.emb, o.emb) and torch.equal(w.head, o.head)
    for a, b in zip(w.blocks, o.blocks):
        assert torch.equal(a.att.rkvWt, b.att.rkvWt)
        assert torch.equal(a.att.oWt, b.att.oWt)
        assert torch.equal(a.att.g1t, b.att.g1t)
        assert torch.equal(a.ffn.kWt, b.ffn.kWt) and torch.equal(a.ffn.vWt, b.ffn.vWt)
    d = model_dims(w)
    assert (d.n_layer, d.n_embd, d.n_ffn, d.vocab) == (3, 256, 1024, 512)
    assert (d.rank_w, d.rank_a, d.rank_v, d.rank_g) == (32, 32, 16, 64)


def test_weight_loads_checkpoint_file(tmp_path):
    sd = make_random_state_dict("tiny", seed=1, dtype=torch.float32)
    p = tmp_path / "ck.pth"
    torch.save(sd, p)
    w = RWKV7Weight(str(p), device="cpu", dtype=torch.float16)
    assert w.L == 3 and w.dtype == torch.float16 and w.head.dtype == torch.float16


def test_weight_loads_bf16_checkpoint_as_fp16(tmp_path):
    """Real checkpoints are bf16 (src/rwkv_tl/weight.py:161-169): the loader
    converts every tensor to the target dtype once, so a bf16 file loads to
    exactly the fp16 rounding of its values, and LN0 is applied to emb in
    fp16 (the same path as an fp16 file of those values)."""
    sd32 = make_random_state_dict("tiny", seed=2, dtype=torch.float32)
    sd_bf16 = {k: v.to(torch.bfloat16) for k, v in sd32.items()}
    p = tmp_path / "ck_bf16.pth"
    torch.save(sd_bf16, p)
    w = RWKV7Weight(str(p), device="cpu", dtype=torch.float16)
    ref = RWKV7Weight.from_state_dict({k: v.to(torch.float16) for k, v in sd_bf16.items()}, device="cpu")
    assert w.head.dtype == torch.float16
    assert torch.equal(w.head, sd_bf16["head.weight"].to(torch.float16))
    assert torch.equal(w.emb, ref.emb)
    for a, b in zip(w.blocks, ref.blocks):
        assert torch.equal(a.att.rkvWt[1], b.att.rkvWt[1]) and torch.equal(a.ffn.vWt, b.ffn.vWt)


# Oracle sampling pinned by the known answers of the reference's
# test/test_sampling.py:11-59 and by the filters' definitions.
def test_sampling_ref_greedy_argmax():
    logits = torch.tensor([1.0, 2.0, 0.5, 3.0])
    assert S.sample_logits_ref(logits).item() == 3
    assert S.sample_logits_ref(logits, temperature=0.0).item() == 3
    assert S.sample_logits_ref(logits, temperature=-1.0).item() == 3


def test_sampling_ref_top_k_one_is_greedy():
    torch.manual_seed(0)
    logits = torch.randn(100)
    for _ in range(20):
        assert S.sample_logits_ref(logits, temperature=1.0, top_k=1).item() == int(logits.argmax())


def test_sampling_ref_repetition_penalty_flips_near_tie():
    logits = torch.tensor([0.5, 0.4])
    assert S.sample_logits_ref(logits, temperature=1.0, top_k=1).item() == 0
    got = S.sample_logits_ref(logits, temperature=1.0, top_k=1, repetition_penalty=2.0, seen=torch.tensor([0]))
    assert got.item() == 1


def test_sampling_ref_range_and_shape():
    torch.manual_seed(0)
    logits = torch.randn(100)
    for _ in range(20):
        assert 0 <= S.sample_logits_ref(logits, temperature=1.0, top_k=50, top_p=0.9).item() < 100
    for temperature in (None, 0.0, 1.0):
        t = S.sample_logits_ref(torch.randn(65536), temperature=temperature)
        assert t.numel() == 1 and 0 <= int(t) < 65536
    assert S.sample_logits_ref(torch.randn(3, 10), temperature=1.0, top_p=0.5).shape == (3,)


def test_sampling_ref_top_p_keeps_smallest_nucleus():
    # probabilities 0.5, 0.3, 0.2: top_p 0.6 keeps the first two only
    logits = torch.log(torch.tensor([0.5, 0.3, 0.2]))
    torch.manual_seed(0)
    draws = {int(S.sample_logits_ref(logits, temperature=1.0, top_p=0.6)) for _ in range(200)}
    assert draws == {0, 1}


@pytest.mark.parametrize("top_k,top_p", [(5, 1.0), (0, 0.5), (0, 0.9), (7, 0.8), (1, 0.3), (40, 0.05)])
def test_sampling_ref_filters_match_definitions(top_k, top_p):
    g = torch.Generator().manual_seed(top_k * 100 + int(top_p * 10))
    for temperature in (0.7, 1.3):
        logits = torch.randn(40, generator=g) * 2
        l = S.filtered_logits_ref(logits, temperature=temperature, top_k=top_k, top_p=top_p)
        got = [bool(v) for v in torch.isfinite(l)]
        want = S.kept_mask_brute((logits.float() / temperature).tolist(), top_k, top_p)
        assert got == want


def test_philox_known_answers():
    """Random123 known-answer vectors of philox4x32 with 10 rounds."""
    assert S.philox4x32_10((0, 0, 0, 0), (0, 0)) == (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)
    f = 0xFFFFFFFF
    assert S.philox4x32_10((f, f, f, f), (f, f)) == (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)
    assert S.philox4x32_10((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0)) == (
        0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1,
    )


def test_draw_ref_is_inverse_cdf():
    probs = __import__("numpy").array([0.1, 0.0, 0.6, 0.3])
    for off in range(50):
        tok, t, cdf = S.draw_ref(probs, seed=12345, offset=off)
        assert probs[tok] > 0 and (tok == 0 or cdf[tok - 1] <= t) and t < cdf[tok]


def test_sample_logits_rejects_cpu_tensors():
    with pytest.raises(ValueError):
        sample_logits(torch.randn(10))


def test_make_rwkv7_backends():
    assert make_rwkv7(torch.device("cuda"), backend="bf16", use_graph=False).__name__ == "RWKV7HIPBF16"
    with pytest.raises(ValueError):
        make_rwkv7(torch.device("cuda"), backend="torch")
    with pytest.raises(ValueError):
        make_rwkv7(torch.device("cuda"), backend="nope")
    with pytest.raises(ValueError):
        make_rwkv7(torch.device("cpu"))
    cls = make_rwkv7(torch.device("cuda"), backend="fp16")
    assert cls.__name__ == "HIPGraphRWKV7HIP"
    assert make_rwkv7(torch.device("cuda"), backend="int8", use_graph=False).__name__ == "RWKV7HIPInt8"
    assert make_rwkv7(torch.device("cuda"), use_graph=False).__name__ == "RWKV7HIP"
    # "auto" is the bfloat16 model, as demo/__init__.py:98-104 picks RWKV7BF16 on sm >= 80
    assert make_rwkv7(torch.device("cuda"), backend="auto", use_graph=False).__name__ == "RWKV7HIPBF16"
    assert make_rwkv7(torch.device("cuda"), backend="auto").__name__ == "HIPGraphRWKV7HIPBF16"


def test_quantize_rows_i8_bounds():
    """Per-row symmetric int8: every element within half a step of its row's
    scale, the row's largest |element| maps to +-127, an all-zero row gets
    scale 0, and a row's scale follows its own largest element only."""
    g = torch.Generator().manual_seed(5)
    W = torch.randn(40, 300, generator=g).half()
    W[3] = 0
    W[7, 11] = 40.0  # an outlier widens only its own row's step
    q, s = quantize_rows_i8(W)
    assert q.dtype == torch.int8 and q.shape == W.shape and s.dtype == torch.float32 and s.shape == (40,)
    w = W.float()
    assert float(s[3]) == 0.0 and int(q[3].abs().max()) == 0
    nz = torch.arange(40) != 3
    assert torch.equal(q[nz].abs().amax(1).int(), torch.full((39,), 127, dtype=torch.int32))
    assert torch.allclose(s, w.abs().amax(1) / 127)
    err = (w - q.float() * s[:, None]).abs()
    assert bool((err <= s[:, None] * 0.5 + 1e-6 * w.abs().amax(1, keepdim=True)).all())  # + f32 rounding
    assert float(s[7]) == pytest.approx(40.0 / 127) and float(s[8]) < 0.05
    # a row that is an exact multiple of its step round-trips exactly
    e = torch.arange(-127, 128, dtype=torch.float32)[None, :] * 0.5
    qe, se = quantize_rows_i8(e)
    assert float(se[0]) == 0.5 and torch.equal(qe[0].float(), torch.arange(-127, 128, dtype=torch.float32))
