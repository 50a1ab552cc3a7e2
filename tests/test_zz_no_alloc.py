"""``rwkv7_decode_noalloc``: the batch-1 decode entry point that allocates nothing.

It runs the same persistent decode kernel as ``rwkv7_decode`` with the
kernel's exchange region in the library's static device array instead of the
caller's workspace, so on identical inputs its logits and state must equal
``rwkv7_decode``'s bit for bit. Checked through the C ABI on two calls in a
row on the 0.1B model, then on the smaller ``tiny`` model (the array is laid
out again for the other sizes), each against ``rwkv7_decode`` on a copy of the
same state.
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
