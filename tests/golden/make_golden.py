"""Write golden vectors from rwkv-tl's own pure-torch path (run in the build container).

The reference has no golden vectors or fixtures; the composition of its model
(``demo/rwkv7_torch.py:67-257``: op order, fp16 rounding points, v_first
threading, token shift) and the ``RWKV7Weight`` load transforms
(``src/rwkv_tl/weight.py:155-184``) are only pinned by running that code. This
script imports exactly those files from a local checkout of the reference and
records their outputs on seeded random-init checkpoints. The reference is not
needed anywhere else: tests read only the files this script writes.

Import mechanics (no arithmetic is touched):

* ``src/rwkv_tl/state.py:3`` imports ``typing.Self`` (Python >= 3.11); on 3.10
  ``typing.Self`` is pointed at ``typing_extensions.Self`` before the import.
* ``demo/__init__.py`` pulls in the TileLang kernels, which are not installed,
  so a bare ``demo`` package object is registered and only
  ``demo/sampling.py``, ``demo/_rwkv7_abc.py`` and ``demo/rwkv7_torch.py`` are
  loaded from it.

Outputs (``tests/golden/``):

* ``tiny_fp32.safetensors`` / ``tiny_fp16.safetensors``: the ``tiny`` shape
  (L=3, C=256, F=1024, V=512, ranks w/a/v/g 32/32/16/64), seed 0; per-step
  decode logits, final decode state, prefill state and forward logits.
* ``c1_0p1b.json``: config C1 (0.1B, fp32, seed 0): prompt decoded token by
  token from zero state, then 32 greedy steps; ids, per-step logit digests and
  final state norms.
* ``manifest.json``: shapes, seeds, token ids and weight digests.

Usage: ``python tests/golden/make_golden.py [--reference /root/reference]``.
"""

from __future__ import annotations

import argparse
import importlib
import json
import sys
import tempfile
import types
import typing
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO / "rwkv-tl_amd"))

from rwkv_tl_amd.checkpoint import (  # noqa: E402
    SHAPES,
    make_random_state_dict,
    save_checkpoint,
    state_dict_digest,
)

TINY_DECODE_TOKENS = 12
C1_PROMPT = 8
C1_GREEDY = 32


def load_reference(ref: Path):
    """Import the reference's pure-torch model without its TileLang kernels."""
    import typing_extensions

    if not hasattr(typing, "Self"):
        typing.Self = typing_extensions.Self  # type: ignore[attr-defined]
    sys.path.insert(0, str(ref / "src"))
    demo = types.ModuleType("demo")
    demo.__path__ = [str(ref / "demo")]  # type: ignore[attr-defined]
    sys.modules["demo"] = demo
    state_mod = importlib.import_module("rwkv_tl.state")
    weight_mod = importlib.import_module("rwkv_tl.weight")
    torch_mod = importlib.import_module("demo.rwkv7_torch")
    return state_mod.State, weight_mod.RWKV7Weight, torch_mod.RWKV7Torch


def _lcg_tokens(n: int, vocab: int) -> list[int]:
    # test/test_forward.py:25-26 recipe, folded into the vocab
    return [((i * 1103515245 + 12345) % 65536) % vocab for i in range(n)]


def _flat_state(S, prefix: str) -> dict[str, torch.Tensor]:
    out = {}
    for i, (t, c) in enumerate(zip(S.tmix, S.cmix)):
        out[f"{prefix}.{i}.tmix_x"] = t["x"].float().clone()
        out[f"{prefix}.{i}.rnn"] = t["rnn"].float().clone()
        out[f"{prefix}.{i}.cmix_x"] = c["x"].float().clone()
    return out


def tiny_vectors(State, RWKV7Weight, RWKV7Torch, dtype: torch.dtype, ckpt: str):
    from safetensors.torch import save_file

    s = SHAPES["tiny"]
    toks = _lcg_tokens(TINY_DECODE_TOKENS, s.vocab)
    w = RWKV7Weight(ckpt, device="cpu", dtype=dtype)
    model = RWKV7Torch(w, is_torch_compile=False)
    # LN0 at load (weight.py:175): 32 rows verbatim plus per-row sums of all rows
    out: dict[str, torch.Tensor] = {
        "emb_ln0_head": w.emb[:32].float().clone(),
        "emb_ln0_rowsum": w.emb.double().sum(dim=1).clone(),
    }

    S = State(w.L, w.C, 64, device="cpu", dtype=dtype)
    logits = []
    for t in toks:
        lg, S = model.decode(torch.tensor([t]), S)
        logits.append(lg.float().clone())
    out["decode_logits"] = torch.stack(logits)
    out.update(_flat_state(S, "decode_state"))

    S = State(w.L, w.C, 64, device="cpu", dtype=dtype)
    model.prefill(torch.tensor(toks[:-1]), S)
    out.update(_flat_state(S, "prefill_state"))
    lg, S = model.decode(torch.tensor([toks[-1]]), S)
    out["prefill_then_decode_logits"] = lg.float().clone()

    S = State(w.L, w.C, 64, device="cpu", dtype=dtype)
    lg, S = model.forward(torch.tensor(toks), S)
    out["forward_logits"] = lg.float().clone()

    name = "tiny_fp32" if dtype == torch.float32 else "tiny_fp16"
    save_file({k: v.contiguous() for k, v in out.items()}, str(HERE / f"{name}.safetensors"))
    return toks


def c1_vectors(State, RWKV7Weight, RWKV7Torch, ckpt: str, prompt_seed: int = 1):
    s = SHAPES["0.1b"]
    gen = torch.Generator(device="cpu").manual_seed(prompt_seed)
    prompt = torch.randint(0, s.vocab, (C1_PROMPT,), generator=gen).tolist()
    w = RWKV7Weight(ckpt, device="cpu", dtype=torch.float32)
    model = RWKV7Torch(w, is_torch_compile=False)
    S = State(w.L, w.C, 64, device="cpu", dtype=torch.float32)
    steps = []
    lg = None
    for t in prompt:
        lg, S = model.decode(torch.tensor([t]), S)
    ids = []
    for _ in range(C1_GREEDY):
        assert lg is not None
        top = torch.topk(lg, 5)
        nxt = int(lg.argmax())
        steps.append(
            {
                "top5_ids": top.indices.tolist(),
                "top5_vals": [float(v) for v in top.values],
                "sum": float(lg.double().sum()),
                "l2": float(lg.double().norm()),
            }
        )
        ids.append(nxt)
        lg, S = model.decode(torch.tensor([nxt]), S)
    norms = {
        f"layer{i}": {
            "rnn_l2": float(t["rnn"].double().norm()),
            "tmix_x_l2": float(t["x"].double().norm()),
            "cmix_x_l2": float(c["x"].double().norm()),
        }
        for i, (t, c) in enumerate(zip(S.tmix, S.cmix))
    }
    return {"prompt": prompt, "prompt_seed": prompt_seed, "greedy_ids": ids, "steps": steps, "final_state": norms}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--skip-c1", action="store_true")
    args = ap.parse_args()
    torch.manual_seed(0)
    State, RWKV7Weight, RWKV7Torch = load_reference(Path(args.reference))

    manifest: dict = {"torch": torch.__version__}
    with tempfile.TemporaryDirectory() as tmp:
        sd = make_random_state_dict("tiny", seed=0, dtype=torch.float32)
        ck = str(Path(tmp) / "tiny.pth")
        save_checkpoint(sd, ck)
        toks = None
        for dt in (torch.float32, torch.float16):
            toks = tiny_vectors(State, RWKV7Weight, RWKV7Torch, dt, ck)
        manifest["tiny"] = {
            "shape": SHAPES["tiny"].__dict__,
            "seed": 0,
            "weights_fp32_sha256": state_dict_digest(sd),
            "tokens": toks,
        }
        if not args.skip_c1:
            sd = make_random_state_dict("0.1b", seed=0, dtype=torch.float32)
            ck = str(Path(tmp) / "c1.pth")
            save_checkpoint(sd, ck)
            manifest["c1"] = {
                "shape": SHAPES["0.1b"].__dict__,
                "seed": 0,
                "weights_fp32_sha256": state_dict_digest(sd),
            }
            del sd
            c1 = c1_vectors(State, RWKV7Weight, RWKV7Torch, ck)
            (HERE / "c1_0p1b.json").write_text(json.dumps(c1, indent=1) + "\n")
    (HERE / "manifest.json").write_text(json.dumps(manifest, indent=1) + "\n")
    print("wrote", sorted(p.name for p in HERE.iterdir() if p.suffix in (".json", ".safetensors")))


if __name__ == "__main__":
    main()
