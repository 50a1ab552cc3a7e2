"""Write the fp16-oracle ("ref16") logits of config C4 (run in the build container).

The oracle's fp16 path runs every torch operation in float16 on the CPU, which
takes minutes per 128-token prefill on CPUs without a fast half-precision
path (the GPU box's host is one), so the C4 test compares the HIP path with
ref16 through this fixture instead of recomputing it there. It holds, for
every C4 case (0.4B, seed-0 fp16 weights, B x T in 1x8, 1x32, 1x64, 1x128,
1x512, 8x8, 16x16) and the rows 0 and B-1 of the batch, the logits of the first
decode step after the prefill: the 64 largest and 2048 seeded random entries
(index, value), plus the first and last prompt ids as a check that the test
draws the same inputs.

Inputs follow tests/test_gpu_configs.py: ``torch.Generator().manual_seed(1000
* B + T)``, then ``randint(0, V, (B, T))`` for the prompt and ``randint(0, V,
(steps, B))`` for the decode tokens (64 steps for B = 1, 16 otherwise).

Usage: ``python tests/golden/make_c4_ref16.py`` (writes ``c4_ref16.safetensors``).
"""

from __future__ import annotations

import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
for p in (REPO / "rwkv-tl_amd", REPO):
    sys.path.insert(0, str(p))

from oracle import rwkv7_ref as R  # noqa: E402
from rwkv_tl_amd.checkpoint import make_random_state_dict  # noqa: E402
from rwkv_tl_amd.weight import RWKV7Weight  # noqa: E402

C4_CASES = [(1, 8), (1, 32), (1, 64), (1, 128), (1, 512), (8, 8), (16, 16)]
TOPK = 64
NRAND = 2048


def inputs(B: int, T: int, V: int):
    g = torch.Generator().manual_seed(1000 * B + T)
    prompt = torch.randint(0, V, (B, T), generator=g)
    steps = 64 if B == 1 else 16
    toks = torch.randint(0, V, (steps, B), generator=g)
    return prompt, toks


def main() -> None:
    torch.set_num_threads(max(1, torch.get_num_threads()))
    sd = make_random_state_dict("0.4b", seed=0, dtype=torch.float16)
    w = RWKV7Weight.from_state_dict(sd, device="cpu", dtype=torch.float16)
    ref16 = R.Weights.from_emb(sd, w.emb, torch.float16)
    V = w.head.shape[0]
    out: dict[str, torch.Tensor] = {}
    for B, T in C4_CASES:
        prompt, toks = inputs(B, T, V)
        for b in sorted({0, B - 1}):
            st = R.new_state(w.L, w.C, dtype=torch.float16)
            R.prefill(ref16, prompt[b], st)
            lg, _ = R.decode(ref16, toks[0, b : b + 1], st)
            lg = lg.float()
            g = torch.Generator().manual_seed(7 * (1000 * B + T) + b)
            idx = torch.cat([torch.topk(lg, TOPK).indices, torch.randint(0, V, (NRAND,), generator=g)])
            key = f"{B}x{T}_row{b}"
            out[f"{key}_idx"] = idx.to(torch.int64).contiguous()
            out[f"{key}_val"] = lg[idx].contiguous()
            out[f"{key}_prompt_ends"] = torch.stack([prompt[b, 0], prompt[b, -1]]).to(torch.int64)
            print(f"{key}: top logit {float(lg.max()):.4f}", flush=True)
    save_file(out, str(HERE / "c4_ref16.safetensors"))


if __name__ == "__main__":
    main()
