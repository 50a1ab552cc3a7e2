"""Benchmark: RWKV7-0.4B fp16 decode (B=1, HIP-graph replay) on one MI355X.

``python bench.py [--gpus 1] [--steps K] [--warmup W]`` prints ONE JSON line.

* A step is one decode token of the 0.4B model (24 layers, C=1024, H=16,
  F=4096, V=65536, LoRA ranks 64/64/32/128), fp16 weights from seed 0, batch
  1, through ``HIPGraph`` replay, token ids drawn uniformly from a seeded
  generator and resident on the device before timing starts. ``value`` is
  ms/token over exactly K timed steps (HIP events on the replay stream,
  bracketed by device synchronisation).
* Extra lines of the same JSON object: decode at batch 16 (ms/step and
  tokens/s), prefill T=128 and T=8 (ms), the roofline of the dominant kernel
  and of the whole step, and the CPU baseline: the oracle's pure-torch fp32
  model (a port of the reference's ``demo/rwkv7_torch.py``) timed on this
  host's cores on a bounded sample of the same decode workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (REPO / "rwkv-tl_amd", REPO):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "RWKV7-0.4B ms/token decode B=1 & prefill T=128 ms; % HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def algorithmic_bytes(shape, batch: int, tokens_per_seq: int, head: bool) -> float:
    """fp16 weights read once + fp32 wkv state read and written + the small
    per-token vectors; intermediates excluded."""
    C, F, V, L, H = shape.n_embd, shape.n_ffn, shape.vocab, shape.n_layer, shape.n_head
    SR = shape.rank_w + shape.rank_a + shape.rank_v + shape.rank_g
    p_layer = 4 * C * C + 2 * C * F + 2 * C * SR + 19 * C  # matrices + per-layer vectors
    weights = 2 * L * p_layer + (2 * V * C if head else 0)
    state = batch * L * (8 * H * 64 * 64 + 8 * C)
    io = batch * tokens_per_seq * 2 * C + (batch * 2 * V if head else 0)
    return float(weights + state + io)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_cuda(fn, iters: int) -> float:
    import torch

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


def cpu_baseline(shape_name: str, steps: int, warmup: int) -> dict:
    """The oracle's fp32 pure-torch decode on the host cores (bounded sample)."""
    import torch

    from oracle import rwkv7_ref as R
    from rwkv_tl_amd.checkpoint import make_random_state_dict

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    sd = make_random_state_dict(shape_name, seed=0, dtype=torch.float16)
    W = R.Weights(sd, torch.float32)
    del sd
    st = R.new_state(W.L, W.C, dtype=torch.float32)
    g = torch.Generator().manual_seed(2)
    toks = torch.randint(0, W.head.shape[0], (steps + warmup,), generator=g)
    with torch.inference_mode():
        for t in toks[:warmup]:
            R.decode(W, t.reshape(1), st)
        t0 = time.perf_counter()
        for t in toks[warmup:]:
            R.decode(W, t.reshape(1), st)
        dt = time.perf_counter() - t0
    cpu_name = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(dt * 1000.0 / steps, 3),
        "unit": "ms/token",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"0.4B fp32 decode B=1, {steps} timed tokens after {warmup} warm-up, from zero state",
        "cpu": cpu_name,
    }


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--cpu-steps", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="only the headline decode line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU only (--gpus {args.gpus} requested): the decode path has no "
            "multi-GPU variant in this build; run with --gpus 1",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch

    from rwkv_tl_amd import SHAPES, HIPGraph, RWKV7HIP, State
    from rwkv_tl_amd.checkpoint import make_random_state_dict
    from rwkv_tl_amd.weight import RWKV7Weight

    dev = torch.device("cuda:0")
    shape = SHAPES["0.4b"]
    log("building 0.4B weights (seed 0)")
    sd = make_random_state_dict("0.4b", seed=0, dtype=torch.float16)
    w = RWKV7Weight.from_state_dict(sd, device=dev, dtype=torch.float16)
    del sd
    model = RWKV7HIP(w, is_torch_compile=False)
    graphed = HIPGraph(model)
    V = shape.vocab
    g = torch.Generator(device="cpu").manual_seed(1)

    # ---- headline: decode B=1 -------------------------------------------------
    K, Wm = args.steps, args.warmup
    toks = torch.randint(0, V, (K + Wm, 1), generator=g).to(dev)
    S = State(w.L, w.C, 64, device=dev)
    log(f"decode B=1: {Wm} warm-up + {K} timed steps")
    for i in range(Wm):
        graphed.decode(toks[i], S)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(Wm, Wm + K):
        logits, S = graphed.decode(toks[i], S)
    end.record()
    torch.cuda.synchronize()
    ms_tok = start.elapsed_time(end) / K
    step_bytes = algorithmic_bytes(shape, 1, 1, head=True)
    step_gbs = step_bytes / (ms_tok * 1e-3) / 1e9

    out: dict = {
        "metric": METRIC,
        "value": round(ms_tok, 5),
        "unit": "ms/token",
        "n_gpus": 1,
        "steps": K,
        "warmup": Wm,
        "ms_per_step": round(ms_tok, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: seeded random-init weights (N(0,0.02)) and uniform random token ids",
        "config": {
            "workload": "RWKV7-0.4B decode B=1, HIP-graph replay (config 3)",
            "layers": shape.n_layer,
            "n_embd": shape.n_embd,
            "vocab": V,
            "batch": 1,
        },
        "tokens_per_s": round(1000.0 / ms_tok, 1),
        "roofline_step": {
            "bound": "hbm",
            "achieved": round(step_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(step_gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
            "alg_bytes_per_step": step_bytes,
        },
    }
    out["roofline"] = dict(out["roofline_step"], kernel="whole decode step (graph replay)")

    if not args.no_extra:
        # ---- decode B=16 ----
        B = 16
        SB = State(w.L, w.C, 64, device=dev, batch=B)
        tb = torch.randint(0, V, (40, B), generator=g).to(dev)
        for i in range(8):
            graphed.decode(tb[i], SB)
        ms16 = time_cuda(lambda it=iter(range(8, 40)): graphed.decode(tb[next(it)], SB), 32)
        b16 = algorithmic_bytes(shape, B, 1, head=True)
        out["decode_b16"] = {
            "ms_per_step": round(ms16, 4),
            "tokens_per_s": round(B * 1000.0 / ms16, 1),
            "hbm_frac": round(b16 / (ms16 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        }
        log(f"decode B=16: {ms16:.4f} ms/step")
        # ---- prefill ----
        pre = {}
        for T in (8, 128):
            tp = torch.randint(0, V, (T,), generator=g).to(dev)
            SP = State(w.L, w.C, 64, device=dev)
            for _ in range(3):
                graphed.prefill(tp, SP)
            ms = time_cuda(lambda: graphed.prefill(tp, SP), 10)
            pb = algorithmic_bytes(shape, 1, T, head=False)
            C, F, L = shape.n_embd, shape.n_ffn, shape.n_layer
            SR = shape.rank_w + shape.rank_a + shape.rank_v + shape.rank_g
            flops = 2.0 * T * L * (4 * C * C + 2 * C * F + 2 * C * SR)
            pre[f"T{T}"] = {
                "ms": round(ms, 4),
                "tokens_per_s": round(T * 1000.0 / ms, 1),
                "hbm_frac": round(pb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 5),
            }
            log(f"prefill T={T}: {ms:.4f} ms")
        out["prefill"] = pre
        out["prefill_T128_ms"] = pre["T128"]["ms"]

    if not args.no_cpu:
        log(f"CPU baseline: {args.cpu_steps} decode steps of the fp32 oracle")
        out["cpu_baseline"] = cpu_baseline("0.4b", args.cpu_steps, 1)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
