"""``RWKV7HIP``: the RWKV7 model on hand-written gfx950 HIP kernels.

Stands in for ``RWKV7FP16`` / ``RWKV7Base`` (``demo/rwkv7_fp16.py:16-25``,
``demo/_rwkv7_base.py:33-310``). Every step is one call into
``librwkv7_hip.so``:

* ``decode`` -> ``rwkv7_decode``: one sequence runs as a single persistent
  kernel (GEMV dot products, grid-wide hand-offs between the stages of each
  layer); 2..16 sequences as the few-row persistent kernel (MFMA on 16-row
  weight blocks); more as the MFMA GEMM path with M = batch.
* ``prefill`` -> ``rwkv7_prefill``: B x T <= 16 rows as the few-row kernel;
  longer prompts as MFMA GEMMs for every projection and a wkv7 scan per head:
  the serial LDS-staged scan (cut into segments from T = 64) below T = 128,
  the chunked scan (16-token chunks on fp32 MFMA) from T = 128.

``decode_path = "kernels"`` selects the multi-launch paths throughout.

There is no CPU or torch fallback: without the library, construction raises.
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from . import _lib
from .model import RWKV7Model
from .state import State
from .weight import RWKV7Weight, pack_device_weights


class RWKV7HIP(RWKV7Model):
    """RWKV7 decode / prefill on MI355X (fp16 weights, fp32 state and accumulation).

    Args:
        w: weights loaded as float16 on a ROCm device (``RWKV7HIPBF16``:
            bfloat16).
        is_torch_compile: accepted for signature compatibility with the
            reference classes and ignored (launch overhead is removed with HIP
            graphs instead, see ``HIPGraph``).
        weight_quant: ``None`` (fp16 weights everywhere) or ``"int8"``: batch-1
            decode streams per-row symmetric int8 copies of the layer matrices
            and the head (f32 row scales, f32 accumulation), about half the
            bytes per token; prefill and batched decode keep the fp16 weights.
        check_errors: after every ``decode`` / ``prefill``, synchronise and
            raise ``HipError`` if a persistent kernel of the step gave up a
            bounded wait (see ``last_error``). Off by default: the check costs
            a host sync per call. ``generate`` always checks once, after its
            final sync.
    """

    # the 16-bit format of the weights, the shift states and the logits
    kernel_dtype = torch.float16

    def __init__(self, w: RWKV7Weight, *, is_torch_compile: bool = True, weight_quant: str | None = None,
                 check_errors: bool = False) -> None:
        super().__init__(w)
        if w.dtype != self.kernel_dtype:
            raise ValueError(f"kernel dtype {self.kernel_dtype} does not match weight dtype {w.dtype}")
        if w.device.type != "cuda":
            raise ValueError(f"RWKV7HIP needs the weights on a ROCm GPU, got {w.device}")
        self._is_torch_compile = is_torch_compile
        if weight_quant not in (None, "int8"):
            raise ValueError(f"weight_quant must be None or 'int8', got {weight_quant!r}")
        self._lib = _lib.load()
        self.weight_quant = weight_quant
        self.dev = pack_device_weights(w, int8=weight_quant == "int8")
        self.V = int(self.dev.dims.vocab)
        self._ws: Tensor | None = None
        self._ws_bytes = 0
        self.check_errors = check_errors
        self._errors_seen = 0  # aborted launches already reported on the current workspace

    # ------------------------------------------------------------------ #
    # buffers and descriptors
    # ------------------------------------------------------------------ #

    def workspace(self, batch: int, seq_len: int) -> Tensor:
        """A scratch buffer big enough for ``batch x seq_len`` (grown, never shrunk).

        A larger request replaces the buffer; a captured HIP graph that still
        points at the old one holds its own reference to it (``HIPGraph``), so
        the old buffer is freed once no graph uses it."""
        need = int(self._lib.rwkv7_workspace_bytes(ctypes.byref(self.dev.dims), batch, seq_len))
        if need < 0:
            raise ValueError(f"unsupported batch={batch} seq_len={seq_len}")
        if self._ws is None or self._ws_bytes < need:
            # zeroed: the decode kernel's hand-off words at its start must not match any tag
            self._ws = torch.zeros(need, dtype=torch.uint8, device=self.w.device)
            self._ws_bytes = need
            self._errors_seen = 0  # the error counter lives in the workspace
        return self._ws

    @property
    def decode_path(self) -> str:
        """``"auto"`` (one persistent kernel per step where the device fits its
        grid: batch-1 decode, and batched decode / prefills of at most 16
        rows) or ``"kernels"`` (the multi-launch GEMV and GEMM paths)."""
        return "kernels" if self.dev.desc.flags & _lib.MODEL_MULTI_LAUNCH_DECODE else "auto"

    @decode_path.setter
    def decode_path(self, path: str) -> None:
        if path not in ("auto", "kernels"):
            raise ValueError(f"decode_path must be 'auto' or 'kernels', got {path!r}")
        flags = self.dev.desc.flags & ~_lib.MODEL_MULTI_LAUNCH_DECODE
        self.dev.desc.flags = flags | (_lib.MODEL_MULTI_LAUNCH_DECODE if path == "kernels" else 0)

    def last_error(self) -> int:
        """Aborted persistent-kernel launches on this model's workspace so far
        (synchronises the current stream). An aborted step wrote NaN logits and
        left the State with only the layers completed before the failure."""
        if self._ws is None:
            return 0
        n = ctypes.c_uint32(0)
        rc = self._lib.rwkv7_workspace_errors(self._ws.data_ptr(), self._ws.numel(), ctypes.byref(n),
                                              _lib.stream_handle())
        _lib.check(rc, "rwkv7_workspace_errors")
        return int(n.value)

    def raise_if_aborted(self) -> None:
        """Raise ``HipError`` if a persistent kernel launch aborted since the
        last check (synchronises the current stream). An aborted decode wrote
        NaN logits; an aborted prefill wrote nothing that shows it, and either
        left the State with only the layers finished before the failure. The
        persistent kernels abort only when a bounded wait gives up, e.g. when
        another process or stream held CUs so that the grid was not resident
        all at once."""
        n = self.last_error()
        if n > self._errors_seen:
            new = n - self._errors_seen
            self._errors_seen = n
            raise _lib.HipError(
                f"{new} persistent kernel launch(es) aborted (a bounded wait gave up); the State holds only the "
                "layers finished before the failure")

    def _check_state(self, S: State) -> None:
        t0 = S[0][0]
        if len(S[0]) != self.L or t0["x"].shape[-1] != self.C:
            raise ValueError(f"state of {len(S[0])} layers x {t0['x'].shape[-1]} does not fit the model")
        if t0["x"].dtype != self.kernel_dtype:
            raise ValueError(f"state dtype {t0['x'].dtype} does not match the model dtype {self.kernel_dtype}")
        if t0["x"].device != self.w.device:
            raise ValueError(f"state on {t0['x'].device}, model on {self.w.device}")

    @staticmethod
    def _batch_of(S: State) -> int:
        return 1 if S[0][0]["rnn"].dim() == 3 else S[0][0]["rnn"].shape[0]

    def _arena_state(self, S: State) -> tuple[State, bool]:
        """``S`` itself if its tensors are intact arena views, else a copy."""
        if isinstance(S, State) and S.arena_intact():
            return S, False
        shadow = State(self.L, self.C, self.N, device=self.w.device, dtype=self.kernel_dtype,
                       batch=None if S[0][0]["rnn"].dim() == 3 else self._batch_of(S))
        shadow.copy_(S)
        return shadow, True

    @staticmethod
    def _desc(S: State) -> _lib.StateDesc:
        tx, rnn, cx = S.arenas
        return _lib.StateDesc(tmix_x=tx.data_ptr(), rnn=rnn.data_ptr(), cmix_x=cx.data_ptr(), batch=S.batch_size)

    def _tokens(self, tokens, shape: tuple[int, ...]) -> Tensor:
        t = torch.as_tensor(tokens)
        if t.numel() != int(torch.Size(shape).numel()):
            raise ValueError(f"expected {shape} token ids, got shape {tuple(t.shape)}")
        if t.dtype not in (torch.int64, torch.int32, torch.int16, torch.uint8):
            raise ValueError(f"token ids must be integers, got {t.dtype}")
        if t.device.type == "cpu" and t.numel() and (int(t.min()) < 0 or int(t.max()) >= self.V):
            raise ValueError(f"token id out of range [0, {self.V})")
        return t.to(device=self.w.device, dtype=torch.int64).reshape(shape).contiguous()

    # ------------------------------------------------------------------ #
    # raw steps (also what HIPGraph captures)
    # ------------------------------------------------------------------ #

    def decode_launches(self, batch: int) -> int:
        """Kernel launches of one decode step with logits (1: a single persistent kernel)."""
        return int(self._lib.rwkv7_decode_launches(ctypes.byref(self.dev.desc), batch, 1))

    def f32_activations(self, batch: int, seq_len: int) -> bool:
        """Whether a step of ``batch`` x ``seq_len`` tokens keeps fp32-grade
        activations (False only for prefills long enough to take the large-M
        GEMM path, whose operands are rounded to 16 bits)."""
        r = int(self._lib.rwkv7_step_f32_activations(ctypes.byref(self.dev.desc), batch, seq_len))
        if r < 0:
            raise ValueError(f"unsupported batch={batch} seq_len={seq_len}")
        return r == 1

    def decode_into(self, tok: Tensor, S: State, logits: Tensor | None) -> None:
        """One decode step: ``tok`` int64 [B] on device, ``logits`` [B, V] of the model's dtype, or None."""
        B = S.batch_size
        ws = self.workspace(B, 1)
        sd = self._desc(S)
        rc = self._lib.rwkv7_decode(
            ctypes.byref(self.dev.desc), ctypes.byref(sd), tok.data_ptr(),
            None if logits is None else logits.data_ptr(), ws.data_ptr(), ws.numel(),
            _lib.stream_handle(),
        )
        _lib.check(rc, "rwkv7_decode")

    def prefill_into(self, tok: Tensor, S: State) -> None:
        """Prefill ``tok`` int64 [B, T] on device into ``S``."""
        B, T = tok.shape
        ws = self.workspace(B, T)
        sd = self._desc(S)
        rc = self._lib.rwkv7_prefill(
            ctypes.byref(self.dev.desc), ctypes.byref(sd), tok.data_ptr(), T, ws.data_ptr(),
            ws.numel(), _lib.stream_handle(),
        )
        _lib.check(rc, "rwkv7_prefill")

    # ------------------------------------------------------------------ #
    # RWKV7Model interface
    # ------------------------------------------------------------------ #

    def decode(self, token: Tensor, S: State) -> tuple[Tensor, State]:
        """Advance one token per sequence; logits ``[V]`` (or ``[B, V]`` for a batched state)."""
        self._check_state(S)
        B = self._batch_of(S)
        tok = self._tokens(token, (B,))
        run, shadow = self._arena_state(S)
        logits = torch.empty(B, self.V, dtype=self.kernel_dtype, device=self.w.device)
        self.decode_into(tok, run, logits)
        if shadow:
            _copy_into(S, run)
        if self.check_errors:
            self.raise_if_aborted()
        return (logits[0] if S[0][0]["rnn"].dim() == 3 else logits), S

    def prefill(self, tokens: Tensor, S: State) -> State:
        """Consume ``tokens`` (``[T]``, or ``[B, T]`` for a batched state) in place."""
        self._check_state(S)
        tokens = torch.as_tensor(tokens)
        if tokens.numel() == 0:
            raise RuntimeError("prefill received an empty token sequence")
        batched = S[0][0]["rnn"].dim() == 4
        B = self._batch_of(S)
        if batched:
            if tokens.ndim != 2 or tokens.shape[0] != B:
                raise ValueError(f"Expected [{B}, T] token ids for a batch-{B} state, got {tuple(tokens.shape)}")
            shape = (B, tokens.shape[1])
        else:
            if tokens.ndim != 1:
                raise ValueError(f"Expected 1D token sequence, got {tokens.shape}")
            shape = (1, tokens.shape[0])
        tok = self._tokens(tokens, shape)
        run, shadow = self._arena_state(S)
        self.prefill_into(tok, run)
        if shadow:
            _copy_into(S, run)
        if self.check_errors:
            self.raise_if_aborted()
        return S


def _copy_into(dst, src: State) -> None:
    """Copy ``src`` into any ``(tmix, cmix)`` state of the same shape."""
    for ds, ss in zip(dst[0] + dst[1], src[0] + src[1]):
        for k in ds:
            ds[k].copy_(ss[k])


class RWKV7HIPBF16(RWKV7HIP):
    """The bfloat16 model (``demo/rwkv7_bf16.py:18-27``): bfloat16 weights as
    loaded (``RWKV7Weight(path, dtype=torch.bfloat16)``, no conversion),
    bfloat16 shift states and logits, bf16 MFMA operands in the GEMMs; fp32
    arithmetic and wkv state as in the float16 model."""

    kernel_dtype = torch.bfloat16


class RWKV7HIPInt8(RWKV7HIP):
    """``RWKV7HIP`` whose batch-1 decode streams int8 weights (``weight_quant="int8"``)."""

    def __init__(self, w: RWKV7Weight, *, is_torch_compile: bool = True, check_errors: bool = False) -> None:
        super().__init__(w, is_torch_compile=is_torch_compile, weight_quant="int8", check_errors=check_errors)
