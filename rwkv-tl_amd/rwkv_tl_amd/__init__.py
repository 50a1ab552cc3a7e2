"""rwkv_tl_amd: RWKV7 inference on AMD Instinct MI355X (gfx950) with hand-written HIP kernels.

Drop-in for the GPU path of yuyi2439/rwkv-tl:

* ``State``, ``RWKV7Weight``, ``LNWeight`` -- ``rwkv_tl.state`` / ``rwkv_tl.weight``
* ``RWKV7Model`` -- ``demo._rwkv7_abc.RWKV7Model`` (decode / prefill / forward / generate)
* ``RWKV7HIP`` -- the HIP model (stands in for ``demo.rwkv7_fp16.RWKV7FP16``)
* ``HIPGraph`` / ``make_graph_cls`` -- ``demo.cuda_graph.CUDAGraph`` / ``make_graph_cls``
* ``make_rwkv7`` -- ``demo.make_rwkv7``
* ``kernels`` -- the operator-level API of ``rwkv_tl.kernels.fp16``
* ``sample_logits`` -- ``demo.sampling.sample_logits`` (one HIP kernel launch)
* ``operators`` -- ``torch.ops.rwkv_tl.*`` (``rwkv_tl.operators``), registered on import
* ``tokenizer.Tokenizer`` -- ``rwkv_tl.tokenizer.Tokenizer``
"""

from __future__ import annotations

import torch

from . import operators  # noqa: F401  (registers torch.ops.rwkv_tl.*, as src/rwkv_tl/__init__.py:10 does)
from .checkpoint import SHAPES, ModelShape, make_random_state_dict
from .hip_graph import HIPGraph, make_graph_cls, wrap_model
from .model import RWKV7Model
from .rwkv7_hip import RWKV7HIP, RWKV7HIPBF16, RWKV7HIPInt8
from .sampling import sample_logits
from .state import State
from .weight import LNWeight, RWKV7Weight

__all__ = [
    "HIPGraph",
    "LNWeight",
    "ModelShape",
    "RWKV7HIP",
    "RWKV7HIPBF16",
    "RWKV7HIPInt8",
    "RWKV7Model",
    "RWKV7Weight",
    "SHAPES",
    "State",
    "make_graph_cls",
    "make_random_state_dict",
    "make_rwkv7",
    "sample_logits",
    "wrap_model",
]

# Backend names of demo/__init__.py:81-120. The float16 names map to the HIP
# model; the NVIDIA-specific variants (mx450, rtx3060) have no meaning on
# MI355X and are accepted as aliases so existing scripts keep working. "auto"
# picks the bfloat16 model, as demo/__init__.py:98-104 does on every GPU of
# compute capability 8.0 or newer (the class an MI355X corresponds to).
_HIP_BACKENDS = ("tuned", "fp16", "hip", "rtx3060", "mx450")


def make_rwkv7(
    device: torch.device | str,
    *,
    backend: str = "tuned",
    use_graph: bool = True,
    device_name: str | None = None,
) -> type[RWKV7Model]:
    """Pick the model class for ``device`` (``demo/__init__.py:43-78``).

    Returns ``RWKV7HIP`` wrapped in ``HIPGraph`` when ``use_graph`` (the
    default) and the device is a GPU; ``backend="bf16"`` returns
    ``RWKV7HIPBF16`` (bfloat16 weights, as ``demo/__init__.py:104-105`` picks
    ``RWKV7BF16``), ``backend="auto"`` the same bfloat16 class (the
    reference's choice for every GPU of compute capability 8.0 or newer,
    ``demo/__init__.py:98-104``), and ``backend="int8"`` ``RWKV7HIPInt8``
    (batch-1 decode on per-row int8 weights). ``backend="torch"`` raises: the
    pure-torch reference model is a test oracle here, not a product backend.
    """
    device = torch.device(device)
    if backend == "torch":
        raise ValueError("backend 'torch' is not provided: the pure-torch model is only a test oracle here")
    names = _HIP_BACKENDS + ("auto", "bf16", "int8")
    if backend not in names:
        raise ValueError(f"unknown backend {backend!r} (expected one of {', '.join(names)})")
    if device.type != "cuda":
        raise ValueError(f"RWKV7HIP runs on a ROCm GPU; got device {device}")
    cls = {"auto": RWKV7HIPBF16, "bf16": RWKV7HIPBF16, "int8": RWKV7HIPInt8}.get(backend, RWKV7HIP)
    return make_graph_cls(cls) if use_graph else cls
