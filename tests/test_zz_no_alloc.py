"""``rwkv7_decode_noalloc``: the batch-1 decode entry point that allocates nothing.

It runs the same persistent decode kernel as ``rwkv7_decode`` with the
kernel's exchange region in the library's static device array instead of the
caller's workspace, so on identical inputs its logits and state must equal
``rwkv7_decode``'s bit for bit. Checked through the C ABI on two calls in a
row on the 0.1B model, then on the smaller ``tiny`` model (the array is laid
out again for the other sizes), each against ``rwkv7_decode`` on a copy of the
same state. A third test mixes the two sizes with a call captured into a HIP
graph: the region's layout check runs on the device, so an eager call of one
size after a captured (or replayed) call of the other still clears it.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from rwkv_tl_amd import RWKV7HIP, State, _lib
from rwkv_tl_amd.checkpoint import make_random_state_dict
from rwkv_tl_amd.weight import RWKV7Weight

pytestmark = pytest.mark.gpu


def _desc(S: State) -> _lib.StateDesc:
    tx, rnn, cx = S.arenas
    return _lib.StateDesc(tmix_x=tx.data_ptr(), rnn=rnn.data_ptr(), cmix_x=cx.data_ptr(), batch=S.batch_size)


def _model(shape: str, cuda) -> RWKV7HIP:
    sd = make_random_state_dict(shape, seed=0, dtype=torch.float16)
    w = RWKV7Weight.from_state_dict(sd, device=cuda, dtype=torch.float16)
    return RWKV7HIP(w, is_torch_compile=False)


def test_decode_noalloc_matches_decode(cuda):
    lib = _lib.load()
    stream = _lib.stream_handle()
    for shape, steps in (("0.1b", 2), ("tiny", 1)):
        print(f"decode_noalloc vs decode: {shape}, {steps} step(s)", flush=True)
        m = _model(shape, cuda)
        if m.decode_launches(1) != 1:
            pytest.skip("the persistent decode kernel does not fit this device")
        V = m.V
        Sa = State(m.L, m.C, 64, device=cuda)
        g = torch.Generator().manual_seed(5)
        prompt = torch.randint(0, V, (6,), generator=g).to(cuda)
        m.prefill(prompt, Sa)  # a non-zero starting state
        Sb = State(m.L, m.C, 64, device=cuda)
        Sb.copy_(Sa)
        ws = m.workspace(1, 1)
        for i in range(steps):
            tok = torch.randint(0, V, (1,), generator=g).to(cuda)
            la = torch.full((1, V), 7.0, dtype=torch.float16, device=cuda)
            lb = torch.full((1, V), -7.0, dtype=torch.float16, device=cuda)
            da, db = _desc(Sa), _desc(Sb)
            rc = lib.rwkv7_decode_noalloc(ctypes.byref(m.dev.desc), ctypes.byref(da), tok.data_ptr(), la.data_ptr(),
                                          stream)
            _lib.check(rc, "rwkv7_decode_noalloc")
            rc = lib.rwkv7_decode(ctypes.byref(m.dev.desc), ctypes.byref(db), tok.data_ptr(), lb.data_ptr(),
                                  ws.data_ptr(), ws.numel(), stream)
            _lib.check(rc, "rwkv7_decode")
            torch.cuda.synchronize()
            assert torch.isfinite(la.float()).all(), f"{shape} step {i}: non-finite logits"
            assert torch.equal(la, lb), f"{shape} step {i}: logits differ"
            for x, y in zip(Sa.arenas, Sb.arenas):
                assert torch.equal(x, y), f"{shape} step {i}: state differs"
        del m


def test_decode_noalloc_rejects_what_it_cannot_run(cuda):
    lib = _lib.load()
    m = _model("tiny", cuda)
    S = State(m.L, m.C, 64, device=cuda, batch=2)
    tok = torch.zeros(2, dtype=torch.int64, device=cuda)
    lg = torch.empty(2, m.V, dtype=torch.float16, device=cuda)
    d = _desc(S)
    rc = lib.rwkv7_decode_noalloc(ctypes.byref(m.dev.desc), ctypes.byref(d), tok.data_ptr(), lg.data_ptr(),
                                  _lib.stream_handle())
    assert rc == 2  # RWKV7_ESHAPE: batch 2
    rc = lib.rwkv7_decode_noalloc(ctypes.byref(m.dev.desc), ctypes.byref(d), tok.data_ptr(), None,
                                  _lib.stream_handle())
    assert rc == 1  # RWKV7_EINVAL: no logits


def test_decode_noalloc_mixes_sizes_with_a_captured_call(cuda):
    """0.1B eager, tiny captured (not yet run), tiny eager, the graph replayed
    twice, 0.1B eager again: every call equals rwkv7_decode on a copy of the
    same state. The captured call lays the region out for its sizes only
    when it is replayed, which the next eager call must see."""
    lib = _lib.load()
    big, small = _model("0.1b", cuda), _model("tiny", cuda)
    if big.decode_launches(1) != 1 or small.decode_launches(1) != 1:
        pytest.skip("the persistent decode kernel does not fit this device")
    g = torch.Generator().manual_seed(11)

    def pair(m):
        Sa = State(m.L, m.C, 64, device=cuda)
        m.prefill(torch.randint(0, m.V, (5,), generator=g).to(cuda), Sa)
        Sb = State(m.L, m.C, 64, device=cuda)
        Sb.copy_(Sa)
        return Sa, Sb

    def reference(m, Sb, tok):
        ws = m.workspace(1, 1)
        lb = torch.empty((1, m.V), dtype=torch.float16, device=cuda)
        db = _desc(Sb)
        rc = lib.rwkv7_decode(ctypes.byref(m.dev.desc), ctypes.byref(db), tok.data_ptr(), lb.data_ptr(),
                              ws.data_ptr(), ws.numel(), _lib.stream_handle())
        _lib.check(rc, "rwkv7_decode")
        return lb

    def noalloc(m, Sa, tok, la):
        da = _desc(Sa)
        rc = lib.rwkv7_decode_noalloc(ctypes.byref(m.dev.desc), ctypes.byref(da), tok.data_ptr(), la.data_ptr(),
                                      _lib.stream_handle())
        _lib.check(rc, "rwkv7_decode_noalloc")

    def same(m, Sa, Sb, la, lb, label):
        torch.cuda.synchronize()
        assert torch.isfinite(la.float()).all(), f"{label}: non-finite logits"
        assert torch.equal(la, lb), f"{label}: logits differ"
        for x, y in zip(Sa.arenas, Sb.arenas):
            assert torch.equal(x, y), f"{label}: state differs"

    Ba, Bb = pair(big)
    Sa, Sb = pair(small)
    tok_big = torch.randint(0, big.V, (1,), generator=g).to(cuda)
    la = torch.empty((1, big.V), dtype=torch.float16, device=cuda)
    print("noalloc: 0.1b eager", flush=True)
    noalloc(big, Ba, tok_big, la)
    same(big, Ba, Bb, la, reference(big, Bb, tok_big), "0.1b eager")

    print("noalloc: tiny captured", flush=True)
    tok_g = torch.zeros(1, dtype=torch.int64, device=cuda)
    lg = torch.empty((1, small.V), dtype=torch.float16, device=cuda)
    Sg = State(small.L, small.C, 64, device=cuda)  # the graph's own state, a copy of Sa before each replay
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        noalloc(small, Sg, tok_g, lg)
    torch.cuda.current_stream().wait_stream(side)

    print("noalloc: tiny eager after the capture", flush=True)
    tok = torch.randint(0, small.V, (1,), generator=g).to(cuda)
    ls = torch.empty((1, small.V), dtype=torch.float16, device=cuda)
    noalloc(small, Sa, tok, ls)
    same(small, Sa, Sb, ls, reference(small, Sb, tok), "tiny eager")

    for rep in range(2):
        print(f"noalloc: tiny replay {rep}, then 0.1b eager", flush=True)
        tok = torch.randint(0, small.V, (1,), generator=g).to(cuda)
        tok_g.copy_(tok)
        Sg.copy_(Sa)
        graph.replay()
        torch.cuda.synchronize()
        lr = reference(small, Sb, tok)
        Sa.copy_(Sg)
        same(small, Sa, Sb, lg, lr, f"tiny replay {rep}")
        tok_big = torch.randint(0, big.V, (1,), generator=g).to(cuda)
        noalloc(big, Ba, tok_big, la)
        same(big, Ba, Bb, la, reference(big, Bb, tok_big), f"0.1b eager after replay {rep}")
