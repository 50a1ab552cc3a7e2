"""Benchmark: RWKV7-0.4B fp16 decode (B=1) and prefill on one MI355X.

``python bench.py [--gpus 1] [--steps K] [--warmup W]`` prints ONE JSON line.

* A step is one decode token of the 0.4B model (24 layers, C=1024, H=16,
  F=4096, V=65536, LoRA ranks 64/64/32/128), fp16 weights from seed 0, batch
  1, called through the ``HIPGraph`` wrapper (which launches a batch-1 step
  directly: it is one persistent kernel, so a graph replay would save
  nothing), token ids drawn uniformly from a seeded generator and resident on
  the device before timing starts. ``value`` is ms/token over exactly K timed
  steps (HIP events on the launch stream, bracketed by device
  synchronisation).
* ``roofline`` is that of the dominant kernel, the persistent decode kernel
  (``decode_mk_kernel``, the whole batch-1 step in one launch): algorithmic
  bytes per launch (fp16 weights and head read once, fp32 wkv state and f16
  shift states read and written, token embedding row and logits) divided by
  its average launch duration, measured with HIP events recorded around each
  launch on the stream it is launched on. ``traffic`` is the HBM bytes per
  launch that ``rocprofv3 --pmc FETCH_SIZE`` / ``WRITE_SIZE`` counted, each
  scaled by what the same counter reads for a copy kernel of known size; it is
  read from the committed summary ``profiles/decode_mk_kernel_traffic.txt``
  (null if absent), which ``--pmc-summary`` writes from the two counter runs.
* Extra keys of the same JSON object: decode at batch 16 (ms/step and
  tokens/s), prefill T=128 and T=8 as flat keys ``prefill_T128_ms``,
  ``prefill_T128_hbm_frac``, ``prefill_T128_mfma_frac`` (and the same for
  T8; prefill through HIP-graph replay for T <= 64), batch-1 decode on int8
  weights (``decode_int8``: the same persistent kernel streaming per-row int8
  matrices, its bytes counted at one byte per int8 weight), batch-1 decode of
  the bfloat16 model (``decode_bf16``), the int8 and any4 weight-only GEMVs
  (``rwkv7_gemv_i8``, ``rwkv7_gemv_any4``) against the f16 GEMV on the head
  matrix (65536 x 1024; average launch time over 100 launches and fraction of
  HBM peak for each),
  the roofline of the whole step as the caller sees it, and the CPU baseline: the oracle's pure-torch fp32
  model (a port of the reference's ``demo/rwkv7_torch.py``) timed on this
  host's cores on a bounded sample of the same decode workload, plus its 1x128
  prefill, with the host's core counts.
* Before anything is timed, a correctness gate (as the reference's benchmark
  has, ``script/benchmark_rwkv7.py:158-182``): the first 8 decode steps of the
  timed model against the fp32 oracle on the same weights and token ids
  (logits 1e-2 abs + 1e-3 rel, wkv state 1e-4 relative); on a mismatch the
  bench prints the gate record and exits non-zero. ``correctness`` in the JSON
  line holds the record.

``python bench.py --generate`` prints a different single JSON line instead:
``generate`` of 128 tokens after a 16-token prompt on the same model and
weights, greedy and with temperature 1 / top-k 50 / top-p 0.9, each step one
decode replay plus one launch of the sampling kernel (``rwkv7_sample``), and
the same loop with the reference's sampling composition in torch operators
(``demo/sampling.py:13-70``) for comparison; plus the sampling kernel's
average launch time (HIP events) at B=1 and B=16.

``python bench.py --timeline`` (after ``python rwkv-tl_amd/build_hip.py
--timeline``) loads the diagnostic library whose persistent kernels stamp the
GPU's 100 MHz real-time counter at the stage boundaries of every layer, runs
0.4B decode at B=1 (``decode_mk_kernel``) and B=16 (``rows_mk_kernel``), and
prints each kernel's per-layer timeline (median over the middle layers of
the median and latest workgroup at each point) and one JSON line.
``python bench.py --hops`` (same library) times the hand-off word alone: pairs
of workgroups on different XCDs or on the same XCD exchange device-scope
tagged words, and the line gives the one-way latency per hop.
``python bench.py --gemm-large`` times the large-M GEMM shapes of the 1.5B
prefill through the C ABI: the plain 16-bit epilogue (hipBLASLt) and relu^2
(the library's large-M kernel), with their fractions of the MFMA peak.

``python bench.py --configs`` prints one more JSON line with the survey's
other measurement configurations, each timed with HIP events after warm-up:
C2 (standalone wkv7 scan, B=8, H=16, T=128, fp32 w and state, f16 r/k/v/a/b),
C4 (0.4B prefill at B x T in 1x8, 1x32, 1x64, 1x128, 1x512, 8x8, 16x16 from a
zero state, then 64 decode steps of the same batch) and C5 (1.5B-shaped
model, ranks 96/96/64/256: prefill 4 x 1024, then decode B=64 for 128
steps), with the algorithmic bytes and FLOPs of each and the fractions of the
HBM and MFMA peaks they reach.

Profiling recipe (the counter runs behind ``traffic``)::

    rocprofv3 --pmc FETCH_SIZE --kernel-trace -f csv -d OUT/fetch -o run -- \
        python bench.py --steps 16 --warmup 4 --no-cpu --no-extra --calib-copy
    rocprofv3 --pmc WRITE_SIZE --kernel-trace -f csv -d OUT/write -o run -- \
        python bench.py --steps 16 --warmup 4 --no-cpu --no-extra --calib-copy
    python bench.py --pmc-summary OUT/fetch OUT/write > profiles/decode_mk_kernel_traffic.txt
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
DOMINANT_KERNEL = "decode_mk_kernel"
TRAFFIC_FILE = REPO / "profiles" / "decode_mk_kernel_traffic.txt"
CALIB_BYTES = 1 << 30  # the calibration copy reads and writes this many bytes


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


def int8_decode_bytes(shape, f16_bytes: float) -> float:
    """Batch-1 decode bytes with int8 weights: every matrix the int8 decode
    streams (r/k/v, LoRA first steps, o, FFN key/value, head) costs one byte
    per element instead of two, plus an f32 scale per row; the LoRA second
    steps and vectors stay as they are."""
    C, F, V, L = shape.n_embd, shape.n_ffn, shape.vocab, shape.n_layer
    SR = shape.rank_w + shape.rank_a + shape.rank_v + shape.rank_g
    elems = L * (4 * C * C + 2 * C * F + C * SR) + V * C
    rows = L * (3 * C + SR + C + F + C) + V
    return float(f16_bytes - elems + 4 * rows)


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


def calib_copy() -> None:
    """A plain copy kernel of known size (CALIB_BYTES read, CALIB_BYTES
    written), run so that counter runs can scale FETCH_SIZE / WRITE_SIZE."""
    import torch

    src = torch.ones(CALIB_BYTES // 2, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def _counter_rows(folder: Path) -> list[dict]:
    import csv

    files = sorted(Path(folder).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {folder}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def _per_dispatch(rows: list[dict], counter: str, name_part: str) -> list[float]:
    """Counter value (KiB) per dispatch of kernels whose name contains name_part."""
    acc: dict[str, float] = {}
    for r in rows:
        if r.get("Counter_Name") == counter and name_part in r.get("Kernel_Name", ""):
            key = r.get("Dispatch_Id") or r.get("Correlation_Id")
            acc[key] = acc.get(key, 0.0) + float(r["Counter_Value"])
    return list(acc.values())


def pmc_summary(fetch_dir: str, write_dir: str) -> str:
    """Text summary of the FETCH_SIZE and WRITE_SIZE runs: per-launch bytes of
    the dominant kernel, each scaled by the calibration copy's reading."""
    import statistics

    f_rows, w_rows = _counter_rows(Path(fetch_dir)), _counter_rows(Path(write_dir))
    out = []
    vals = {}
    for counter, rows in (("FETCH_SIZE", f_rows), ("WRITE_SIZE", w_rows)):
        mk = _per_dispatch(rows, counter, DOMINANT_KERNEL)
        cp = _per_dispatch(rows, counter, "neg_kernel") or _per_dispatch(rows, counter, "elementwise")
        if not mk or not cp:
            raise SystemExit(f"{counter}: no dispatches of {DOMINANT_KERNEL} or of the calibration copy")
        mk_kib, cp_kib = statistics.median(mk), statistics.median(cp)
        factor = (CALIB_BYTES / 1024.0) / cp_kib
        vals[counter] = mk_kib * 1024.0 * factor
        out.append(
            f"{counter}: {DOMINANT_KERNEL} median {mk_kib:.1f} KiB/dispatch over {len(mk)} dispatches; "
            f"calibration copy reads {cp_kib:.1f} KiB for {CALIB_BYTES // 1024} KiB moved -> factor {factor:.4f}; "
            f"scaled {vals[counter]:.0f} B"
        )
    total = vals["FETCH_SIZE"] + vals["WRITE_SIZE"]
    out.append(f"traffic_bytes_per_launch: {total:.0f}")
    return "\n".join(out)


def traffic_from_profile() -> float | None:
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def host_cores() -> dict:
    """Cores of this host: all the OS reports, and those this process may run on."""
    return {"host_logical_cpus": os.cpu_count(), "process_affinity_cpus": len(os.sched_getaffinity(0))}


def cpu_baseline(W, steps: int, warmup: int, prefill_t: int) -> dict:
    """The oracle's fp32 pure-torch decode and prefill on the host cores
    (bounded sample). ``W`` is the oracle's fp32 model (``R.Weights``)."""
    import torch

    from oracle import rwkv7_ref as R

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
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
        tp = torch.randint(0, W.head.shape[0], (prefill_t,), generator=g)
        sp = R.new_state(W.L, W.C, dtype=torch.float32)
        t0 = time.perf_counter()
        R.prefill(W, tp, sp)
        dp = time.perf_counter() - t0
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
        "sample": f"0.4B fp32 decode B=1, {steps} timed tokens after {warmup} warm-up, from zero state; "
                  f"prefill_T{prefill_t}_ms: one 1x{prefill_t} prefill from zero state",
        f"prefill_T{prefill_t}_ms": round(dp * 1000.0, 1),
        "cpu": cpu_name,
        **host_cores(),
    }


def correctness_gate(graphed, ref_w, toks, steps: int) -> dict:
    """The reference's benchmark checks each model against the pure-torch one
    before timing it (script/benchmark_rwkv7.py:158-182,280-284). Here: the
    first ``steps`` decode steps of the timed model, from a zero state, on the
    timed token ids, against the fp32 oracle on the same fp16 weights; logits
    within 1e-2 abs + 1e-3 rel, the fp32 wkv state within 1e-4 relative per
    layer. Returns the record; the caller exits non-zero when it failed."""
    import torch

    from oracle import rwkv7_ref as R
    from rwkv_tl_amd import State

    m = graphed.model
    S = State(m.L, m.C, 64, device=toks.device)
    ref = R.new_state(m.L, m.C, dtype=torch.float16)
    max_d, bad, worst_state = 0.0, 0, 0.0
    with torch.inference_mode():
        for i in range(steps):
            lg, S = graphed.decode(toks[i], S)
            lr, ref = R.decode(ref_w, toks[i].cpu(), ref)
            got, want = lg.float().cpu().reshape(-1), lr.float().reshape(-1)
            d = (got - want).abs()
            max_d = max(max_d, float(d.max()))
            bad += int((d > 1e-2 + 1e-3 * want.abs()).sum()) + int((~torch.isfinite(got)).sum())
    for i in range(m.L):
        x, y = S.tmix[i]["rnn"].cpu().double(), ref[0][i]["rnn"].double()
        worst_state = max(worst_state, float((x - y).norm() / y.norm().clamp_min(1e-30)))
    ok = bad == 0 and worst_state <= 1e-4
    return {"steps": steps, "oracle": "fp32 pure-torch port (oracle/rwkv7_ref.py) on the same fp16 weights",
            "logit_bar": "1e-2 abs + 1e-3 rel", "max_abs_logit_diff": round(max_d, 6), "logits_off": bad,
            "state_bar": 1e-4, "max_state_rel_err": float(f"{worst_state:.3e}"), "pass": ok}


def _torch_ops_sample(l, temperature, top_k, top_p):
    """The reference's sampling composition (demo/sampling.py:52-70) in torch
    operators on the device: the per-token cost the sampling kernel replaces."""
    import torch

    l = l.float() / temperature
    cutoff = torch.topk(l, top_k, dim=-1).values[..., -1:]
    l = torch.where(l >= cutoff, l, torch.full_like(l, float("-inf")))
    probs = torch.softmax(l, dim=-1)
    sp, si = torch.sort(probs, descending=True, dim=-1)
    drop = torch.cumsum(sp, dim=-1) - sp > top_p
    kept = torch.gather(l, -1, si)
    l = l.scatter(-1, si, torch.where(drop, torch.full_like(kept, float("-inf")), kept))
    return torch.multinomial(torch.softmax(l, dim=-1), 1).squeeze(-1)


def _flops(shape, tokens: int, head: bool) -> float:
    C, F, L, V = shape.n_embd, shape.n_ffn, shape.n_layer, shape.vocab
    SR = shape.rank_w + shape.rank_a + shape.rank_v + shape.rank_g
    return 2.0 * tokens * (L * (4 * C * C + 2 * C * F + 2 * C * SR) + (V * C if head else 0))


def _fracs(alg_bytes: float, flops: float, ms: float) -> dict:
    return {
        "alg_bytes": alg_bytes,
        "alg_flops": flops,
        "hbm_frac": round(alg_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
    }


def bench_configs() -> dict:
    import torch

    from rwkv_tl_amd import SHAPES, HIPGraph, RWKV7HIP, State
    from rwkv_tl_amd import _lib
    from rwkv_tl_amd import kernels as K
    from rwkv_tl_amd.checkpoint import make_random_state_dict
    from rwkv_tl_amd.weight import RWKV7Weight

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(1)
    out: dict = {"mode": "configs", "data": "synthetic: seeded random-init weights and uniform random token ids",
                 "unit": "ms"}

    # C2: the wkv7 scan alone
    B, T, H, N = 8, 128, 16, 64
    r, k, v = (torch.randn(B, T, H, N, generator=g).half().to(dev) for _ in range(3))
    w = torch.exp(-torch.exp(torch.randn(B, T, H, N, generator=g) * 0.5 - 0.5)).to(dev)
    kh = torch.nn.functional.normalize(torch.randn(B, T, H, N, generator=g), dim=-1)
    alpha = torch.sigmoid(torch.randn(B, T, H, N, generator=g))
    a, b = (-kh).half().to(dev), (kh * alpha).half().to(dev)
    S0 = (torch.randn(B, H, N, N, generator=g) * 0.1).to(dev)
    S = S0.clone()
    K.wkv7(S, r, w, k, v, a, b)  # first call: device properties, library load
    op_ms = time_cuda(lambda: K.wkv7(S, r, w, k, v, a, b), 20)
    # the same launches through the C ABI with the arguments prepared once: the
    # operator's host-side checks and allocation (tens of microseconds of
    # Python per call) no longer leave the GPU idle between launches
    lib = _lib.load()
    y = torch.empty_like(r)
    args = (S.data_ptr(), r.data_ptr(), w.data_ptr(), 1, k.data_ptr(), v.data_ptr(), a.data_ptr(), b.data_ptr(),
            y.data_ptr(), B, T, H, 0)
    st = _lib.stream_handle()
    nb = int(lib.rwkv7_wkv7_chunked_workspace_bytes(B, T, H))
    ws = torch.empty(nb, dtype=torch.uint8, device=dev)
    chunked = lambda: lib.rwkv7_wkv7_chunked(*args, ws.data_ptr(), nb, st)  # noqa: E731
    serial = lambda: lib.rwkv7_wkv7(*args, st)  # noqa: E731
    _lib.check(chunked(), "rwkv7_wkv7_chunked")
    _lib.check(serial(), "rwkv7_wkv7")
    chunked_ms = time_cuda(chunked, 50)
    serial_ms = time_cuda(serial, 50)
    # the algorithm kernels.wkv7 picks for this shape
    ms = chunked_ms if T >= K.CHUNK_MIN_T and 4 * B * H < K._cus(dev) else serial_ms
    c2_bytes = B * T * H * N * (5 * 2 + 4 + 2) + 2 * 4 * B * H * N * N
    out["C2_wkv7_B8_H16_T128"] = {"ms": round(ms, 4), "serial_ms": round(serial_ms, 4),
                                  "chunked_ms": round(chunked_ms, 4), "op_ms": round(op_ms, 4),
                                  **_fracs(c2_bytes, 9.0 * N * N * B * T * H, ms),
                                  "note": "ms: back-to-back C-ABI launches of the algorithm the operator "
                                          "picks for this shape; serial_ms / chunked_ms: rwkv7_wkv7 / "
                                          "rwkv7_wkv7_chunked; op_ms: through kernels.wkv7 (host checks "
                                          "included); FLOPs are the serial recurrence's VALU count "
                                          "(9 N^2 per head per token)"}
    log(f"C2 wkv7: serial {serial_ms:.4f} ms, chunked {chunked_ms:.4f} ms per launch, {op_ms:.4f} ms per operator call")

    def model_for(name: str):
        sd = make_random_state_dict(name, seed=0, dtype=torch.float16)
        wt = RWKV7Weight.from_state_dict(sd, device=dev, dtype=torch.float16)
        del sd
        m = RWKV7HIP(wt, is_torch_compile=False)
        return wt, m, HIPGraph(m)

    def run_case(shape, wt, m, gm, Bq: int, Tq: int, n_dec: int, tag: str, dec_b: int | None = None) -> None:
        """Prefill Bq x Tq from a zero state, then n_dec decode steps of dec_b
        sequences (default Bq, continuing the prefilled state; otherwise from a
        zero state of dec_b sequences)."""
        V = shape.vocab
        dec_b = dec_b or Bq
        toks = torch.randint(0, V, (Bq, Tq), generator=g).to(dev)
        dec = torch.randint(0, V, (n_dec + 4, dec_b), generator=g).to(dev)
        Sq = State(wt.L, wt.C, 64, device=dev, batch=Bq)
        for _ in range(2):
            m.prefill(toks, Sq)
        torch.cuda.synchronize()
        Sq = State(wt.L, wt.C, 64, device=dev, batch=Bq)
        ms_p = time_cuda(lambda: m.prefill(toks, Sq), 10 if Bq * Tq <= 512 else 3)
        if dec_b != Bq:
            Sq = State(wt.L, wt.C, 64, device=dev, batch=dec_b)
        for i in range(4):
            gm.decode(dec[i], Sq)
        it = iter(range(4, n_dec + 4))
        ms_d = time_cuda(lambda: gm.decode(dec[next(it)], Sq), n_dec)
        out[tag] = {
            "prefill_ms": round(ms_p, 4),
            "prefill_tokens_per_s": round(Bq * Tq * 1000.0 / ms_p, 1),
            "prefill": _fracs(algorithmic_bytes(shape, Bq, Tq, head=False), _flops(shape, Bq * Tq, False), ms_p),
            "decode_batch": dec_b,
            "decode_ms_per_step": round(ms_d, 4),
            "decode_tokens_per_s": round(dec_b * 1000.0 / ms_d, 1),
            "decode": _fracs(algorithmic_bytes(shape, dec_b, 1, head=True), _flops(shape, dec_b, True), ms_d),
        }
        log(f"{tag}: prefill {ms_p:.3f} ms, decode {ms_d:.4f} ms/step")

    shape = SHAPES["0.4b"]
    wt, m, gm = model_for("0.4b")
    for Bq, Tq in ((1, 8), (1, 32), (1, 64), (1, 128), (1, 512), (8, 8), (16, 16)):
        run_case(shape, wt, m, gm, Bq, Tq, 64, f"C4_0.4b_prefill_{Bq}x{Tq}_then_64_decode")
    del wt, m, gm
    torch.cuda.empty_cache()
    shape = SHAPES["1.5b"]
    wt, m, gm = model_for("1.5b")
    run_case(shape, wt, m, gm, 4, 1024, 128, "C5_1.5b_prefill_4x1024_then_decode_B64", dec_b=64)
    return out


def bench_generate() -> dict:
    import torch

    from rwkv_tl_amd import make_rwkv7
    from rwkv_tl_amd.checkpoint import make_random_state_dict
    from rwkv_tl_amd.sampling import Sampler
    from rwkv_tl_amd.weight import RWKV7Weight

    dev = torch.device("cuda:0")
    sd = make_random_state_dict("0.4b", seed=0, dtype=torch.float16)
    w = RWKV7Weight.from_state_dict(sd, device=dev, dtype=torch.float16)
    del sd
    model = make_rwkv7(dev)(w, is_torch_compile=False)
    V, n_new = w.head.shape[0], 128
    prompt = torch.randint(0, V, (16,), generator=torch.Generator().manual_seed(1)).tolist()
    cfgs = {"greedy": dict(), "t1_topk50_topp0.9": dict(temperature=1.0, top_k=50, top_p=0.9)}
    out: dict = {"mode": "generate", "workload": "RWKV7-0.4B generate 128 tokens after a 16-token prompt, B=1",
                 "data": "synthetic: seeded random-init weights and prompt", "unit": "ms/token"}
    for name, kw in cfgs.items():
        model.generate(prompt, model.new_state(), 8, **kw)  # warm-up (graph capture)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        model.generate(prompt, model.new_state(), n_new, **kw)
        out[name] = {"ms_per_token": round((time.perf_counter() - t0) * 1000.0 / n_new, 4)}
        log(f"generate {name}: {out[name]['ms_per_token']} ms/token")
    # the same loop with the torch-operator sampler (first pass: warm-up)
    kw = cfgs["t1_topk50_topp0.9"]
    for n in (8, n_new):
        S = model.new_state()
        S = model.prefill(torch.tensor(prompt[:-1], device=dev), S)
        tok = torch.tensor(prompt[-1], device=dev)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        toks = []
        for _ in range(n):
            logits, S = model.decode(tok, S)
            tok = _torch_ops_sample(logits, **kw)
            toks.append(tok)
        torch.stack(toks).tolist()
    out["t1_topk50_topp0.9_torch_ops"] = {"ms_per_token": round((time.perf_counter() - t0) * 1000.0 / n_new, 4)}
    # the sampling kernel alone, per launch
    for B in (1, 16):
        logits = (torch.randn(B, V, generator=torch.Generator().manual_seed(B)) * 2).half().to(dev)
        res = torch.empty(B, dtype=torch.int64, device=dev)
        for name, kw in cfgs.items():
            smp = Sampler(V, dev, batch=B, **kw)
            for _ in range(10):
                smp(logits, res)
            stream = torch.cuda.current_stream()
            evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(100)]
            for a, b in evs:
                a.record(stream)
                smp(logits, res)
                b.record(stream)
            torch.cuda.synchronize()
            us = 1000.0 * sum(a.elapsed_time(b) for a, b in evs) / len(evs)
            out[name][f"sample_kernel_us_B{B}"] = round(us, 2)
            log(f"sample kernel {name} B={B}: {us:.2f} us")
            if "top_k" in kw:  # the same without the workspace: one workgroup per row
                smp.workspace = None
                for a, b in evs:
                    a.record(stream)
                    smp(logits, res)
                    b.record(stream)
                torch.cuda.synchronize()
                us1 = 1000.0 * sum(a.elapsed_time(b) for a, b in evs) / len(evs)
                out[name][f"sample_kernel_us_B{B}_one_workgroup_per_row"] = round(us1, 2)
                log(f"sample kernel {name} B={B}, one workgroup per row: {us1:.2f} us")
    return out


TIMELINE_LIB = Path(__file__).resolve().parent / "rwkv-tl_amd" / "rwkv_tl_amd" / "librwkv7_hip_timeline.so"
# stamp points of the two persistent kernels (csrc/decode_mk.hip, csrc/rows_mk.hip)
TL_DECODE = ["P1 input ready", "P1 published", "P3 input ready", "P3 published", "P4 input ready",
             "P4 published", "P5 input ready", "P5 published", "P2 input ready (heads)", "P2 published (heads)"]
TL_ROWS = ["P1 start", "P1 input ready", "P1 statistics", "P1 products", "P2 start", "P2 done", "P3 start",
           "P3 input ready", "P3 published", "P4 start", "P4 input ready", "P4 statistics", "P4 products",
           "P4 published", "P5 start", "P5 input ready", "P5 products", "P5 published"]


def _timeline_table(buf, names, groups: int, layers: int, ref_point: int) -> dict:
    """buf [32][1024][24] uint64 stamps (100 MHz). Per layer l in 1 .. layers-2,
    times in us from the earliest stamp of ref_point in that layer; for every
    point the median and the maximum over the workgroups that recorded it,
    then the median of those over the layers; plus the layer period."""
    import numpy as np

    rows = {n: {"median_us": [], "last_us": [], "groups": 0} for n in names}
    period = []
    for l in range(1, layers - 1):
        x = buf[l, :groups, : len(names)].astype(np.int64)
        ref = x[:, ref_point][x[:, ref_point] > 0]
        nxt = buf[l + 1, :groups, ref_point].astype(np.int64)
        nxt = nxt[nxt > 0]
        if ref.size == 0:
            continue
        t0 = ref.min()
        if nxt.size:
            period.append((nxt.min() - t0) / 100.0)
        for i, n in enumerate(names):
            v = x[:, i]
            v = v[v > 0]
            if v.size == 0:
                continue
            v = (v - t0) / 100.0
            rows[n]["median_us"].append(float(np.median(v)))
            rows[n]["last_us"].append(float(v.max()))
            rows[n]["groups"] = int(v.size)
    out = {"layer_period_us": round(float(np.median(period)), 2) if period else None, "points": {}}
    for n in names:
        r = rows[n]
        if r["median_us"]:
            out["points"][n] = {"median_us": round(float(np.median(r["median_us"])), 2),
                                "last_us": round(float(np.median(r["last_us"])), 2), "workgroups": r["groups"]}
    return out


def bench_timeline() -> dict:
    """Stage timelines of the two persistent decode kernels (diagnostic build)."""
    import ctypes

    import numpy as np

    if not TIMELINE_LIB.exists():
        raise SystemExit(f"{TIMELINE_LIB} not built: python rwkv-tl_amd/build_hip.py --timeline")
    os.environ["RWKV7_HIP_LIB"] = str(TIMELINE_LIB)
    import torch

    from rwkv_tl_amd import RWKV7HIP, State, _lib
    from rwkv_tl_amd.checkpoint import make_random_state_dict
    from rwkv_tl_amd.weight import RWKV7Weight

    lib = _lib.load()
    dev = torch.device("cuda:0")
    log("building 0.4B weights (seed 0) for the timeline library")
    sd = make_random_state_dict("0.4b", seed=0, dtype=torch.float16)
    w = RWKV7Weight.from_state_dict(sd, device=dev, dtype=torch.float16)
    del sd
    model = RWKV7HIP(w, is_torch_compile=False)
    g = torch.Generator(device="cpu").manual_seed(1)
    shape = (32, 1024, 24)
    out = {"mode": "timeline", "model": "RWKV7-0.4B fp16", "clock": "GPU real-time counter, 100 MHz",
           "reading": "per layer (middle layers), us from the earliest workgroup at the reference point: "
                      "median_us over the workgroups that record the point, last_us the latest of them; "
                      "medians over the layers"}
    for name, B, fn, names, ref in (("decode_mk_kernel B=1", 1, "rwkv7_timeline_read_decode", TL_DECODE, 0),
                                    ("rows_mk_kernel B=16", 16, "rwkv7_timeline_read_rows", TL_ROWS, 1)):
        S = State(w.L, w.C, 64, device=dev, batch=B)
        for _ in range(12):
            tok = torch.randint(0, w.head.shape[0], (B,), generator=g).to(dev)
            _, S = model.decode(tok, S)
        torch.cuda.synchronize()
        model.raise_if_aborted()
        buf = np.zeros(shape, dtype=np.uint64)
        read = getattr(lib, fn)
        read.argtypes = [ctypes.c_void_p, ctypes.c_int64]
        _lib.check(read(buf.ctypes.data, buf.nbytes), fn)
        tab = _timeline_table(buf, names, shape[1], w.L, ref)
        out[name] = tab
        log(f"{name}: layer period {tab['layer_period_us']} us")
        for n, r in tab["points"].items():
            log(f"  {n:24s} median {r['median_us']:7.2f} us  last {r['last_us']:7.2f} us  ({r['workgroups']} workgroups)")
    return out


def bench_gemm_large(calls: int = 20) -> dict:
    """The large-M GEMM shapes of the 1.5B-shaped prefill (M = B*T = 4096 or
    2048), f16 operands, through the C ABI (kernels.gemm): the plain 16-bit
    epilogue and the relu^2 epilogue (both hipBLASLt's half product; relu^2
    adds the in-place squaring pass), HIP events over `calls` calls after
    warm-up."""
    import torch

    from rwkv_tl_amd import kernels as K

    dev = torch.device("cuda:0")
    peak = MFMA_F16_PEAK_TFLOPS * 1e12
    out = {"mode": "gemm_large", "unit": "us per call", "peak_tflops": MFMA_F16_PEAK_TFLOPS, "shapes": {}}
    for M, N, Kd in ((4096, 8192, 2048), (4096, 2048, 8192), (4096, 6400, 2048), (2048, 8192, 2048)):
        g = torch.Generator(device="cpu").manual_seed(M + N + Kd)
        A = (torch.randn(M, Kd, generator=g) * 0.5).half().to(dev)
        W = (torch.randn(N, Kd, generator=g) * 0.02).half().to(dev)
        row = {}
        for epi in ("f16", "relu2"):
            for _ in range(3):
                K.gemm(A, W, epi)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(calls):
                K.gemm(A, W, epi)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / calls * 1000
            frac = 2.0 * M * N * Kd / (us * 1e-6) / peak
            row[epi] = {"us": round(us, 1), "mfma_frac": round(frac, 3)}
        out["shapes"][f"{M}x{N}x{Kd}"] = row
        log(f"{M}x{N}x{Kd}: f16 {row['f16']['us']} us ({row['f16']['mfma_frac']}), "
            f"relu2 {row['relu2']['us']} us ({row['relu2']['mfma_frac']})")
        del A, W
    return out


def bench_hops(rounds: int = 2008) -> dict:
    """One-way latency of the persistent kernels' hand-off word (device-scope
    store, device-scope poll) between two workgroups on different XCDs and on
    the same XCD, with nothing else running (diagnostic library's probe)."""
    import ctypes

    import numpy as np

    if not TIMELINE_LIB.exists():
        raise SystemExit(f"{TIMELINE_LIB} not built: python rwkv-tl_amd/build_hip.py --timeline")
    os.environ["RWKV7_HIP_LIB"] = str(TIMELINE_LIB)
    import torch

    from rwkv_tl_amd import _lib

    lib = _lib.load()
    fn = lib.rwkv7_probe_hops
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_uint32,
                   ctypes.c_void_p, ctypes.c_void_p]
    dev = torch.device("cuda:0")
    G = torch.cuda.get_device_properties(dev).multi_processor_count // 16 * 16
    out = {"mode": "hops", "workgroups": G, "rounds": rounds,
           "reading": "per workgroup pair (g, g ^ x): rounds of store own word then poll the partner's; "
                      "us per round = one-way hand-off latency; median / min / max over the workgroups"}
    # workgroup g runs on XCD g % 8: partners g ^ 1 and g ^ 4 sit on another XCD, g ^ 8 on the same one
    for name, x in (("other XCD (partner g ^ 1)", 1), ("other XCD (partner g ^ 4)", 4),
                    ("same XCD (partner g ^ 8)", 8)):
        res = []
        for rep in range(3):
            words = torch.zeros(16 * G, dtype=torch.int64, device=dev)
            o = torch.zeros(3 * G, dtype=torch.int64, device=dev)
            _lib.check(fn(words.data_ptr(), G, x, rounds, 1 + rep * rounds, o.data_ptr(), _lib.stream_handle()),
                       "rwkv7_probe_hops")
            torch.cuda.synchronize()
            res.append(o.cpu().numpy().reshape(G, 3))
        a = np.stack(res)
        errs = int(a[:, :, 1].sum())
        xcc = a[0, :, 2]
        same = int(sum(xcc[g] == xcc[g ^ x] for g in range(G)))
        us = a[:, :, 0].astype(np.float64) / (rounds - 8) / 100.0  # 100 MHz ticks
        out[name] = {"us_median": round(float(np.median(us)), 3), "us_min": round(float(us.min()), 3),
                     "us_max": round(float(us.max()), 3), "pairs_on_one_xcc": f"{same}/{G}",
                     "polls_given_up": errs}
        log(f"{name:28s} {out[name]['us_median']:.3f} us per hop (min {out[name]['us_min']:.3f}, "
            f"max {out[name]['us_max']:.3f}); pairs on one XCC {same}/{G}; polls given up {errs}")
    out["xcc_of_workgroups_0_15"] = [int(v) for v in xcc[:16]]
    return out


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--cpu-steps", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="only the headline decode line")
    ap.add_argument("--no-gate", action="store_true", help="skip the correctness gate against the fp32 oracle")
    ap.add_argument("--gate-steps", type=int, default=8, help="decode steps the correctness gate checks")
    ap.add_argument("--calib-copy", action="store_true", help="also run a 1 GiB copy kernel (counter calibration)")
    ap.add_argument("--configs", action="store_true",
                    help="time the survey's C2, C4 and C5 configurations instead (one different JSON line)")
    ap.add_argument("--generate", action="store_true",
                    help="time generate() with the on-device sampler instead (one different JSON line)")
    ap.add_argument("--timeline", action="store_true",
                    help="stage timelines of the persistent decode kernels from the diagnostic library "
                         "(python rwkv-tl_amd/build_hip.py --timeline first; one different JSON line)")
    ap.add_argument("--gemm-large", action="store_true",
                    help="time the large-M GEMM shapes of the 1.5B prefill (hipBLASLt vs the relu^2 kernel)")
    ap.add_argument("--hops", action="store_true",
                    help="hand-off latency between two workgroups on different / the same XCD, from the "
                         "diagnostic library (python rwkv-tl_amd/build_hip.py --timeline first; one JSON line)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarise two rocprofv3 --pmc csv runs and exit (no GPU)")
    args = ap.parse_args()
    if args.pmc_summary:
        print(pmc_summary(*args.pmc_summary))
        return
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU only (--gpus {args.gpus} requested): the decode path has no "
            "multi-GPU variant in this build; run with --gpus 1",
            file=sys.stderr,
        )
        sys.exit(2)
    if args.generate:
        print(json.dumps(bench_generate()), flush=True)
        return
    if args.timeline:
        print(json.dumps(bench_timeline()), flush=True)
        return
    if args.hops:
        print(json.dumps(bench_hops()), flush=True)
        return
    if args.gemm_large:
        print(json.dumps(bench_gemm_large()), flush=True)
        return
    if args.configs:
        print(json.dumps(bench_configs()), flush=True)
        return

    import torch

    from oracle import rwkv7_ref as R
    from rwkv_tl_amd import SHAPES, HIPGraph, RWKV7HIP, State
    from rwkv_tl_amd.checkpoint import make_random_state_dict
    from rwkv_tl_amd.weight import RWKV7Weight

    dev = torch.device("cuda:0")
    shape = SHAPES["0.4b"]
    log("building 0.4B weights (seed 0)")
    sd = make_random_state_dict("0.4b", seed=0, dtype=torch.float16)
    w = RWKV7Weight.from_state_dict(sd, device=dev, dtype=torch.float16)
    # the oracle's fp32 model on the very same weights and embedding rows: the
    # correctness gate's reference and the CPU baseline
    ref_w = R.Weights.from_emb(sd, w.emb.cpu(), torch.float32)
    del sd
    model = RWKV7HIP(w, is_torch_compile=False)
    graphed = HIPGraph(model)
    V = shape.vocab
    g = torch.Generator(device="cpu").manual_seed(1)

    # ---- headline: decode B=1 -------------------------------------------------
    K, Wm = args.steps, args.warmup
    toks = torch.randint(0, V, (K + Wm, 1), generator=g).to(dev)
    gate = None
    if not args.no_gate:
        log(f"correctness gate: {args.gate_steps} decode steps against the fp32 oracle")
        gate = correctness_gate(graphed, ref_w, toks, args.gate_steps)
        log(f"correctness gate: {gate}")
        if not gate["pass"]:
            print(json.dumps({"metric": METRIC, "value": None, "correctness": gate}), flush=True)
            raise SystemExit("correctness gate failed: the decode disagrees with the fp32 oracle")
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

    # ---- dominant kernel: one persistent launch per step, timed per launch --
    if model.decode_launches(1) != 1:
        raise SystemExit("the 0.4B batch-1 decode did not take the one-launch persistent path")
    logits1 = torch.empty(1, V, dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(K)]
    torch.cuda.synchronize()
    for i in range(K):
        evs[i][0].record(stream)
        model.decode_into(toks[Wm + i], S, logits1)
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    kern_us = 1000.0 * sum(a.elapsed_time(b) for a, b in evs) / K
    kern_gbs = step_bytes / (kern_us * 1e-6) / 1e9
    traffic = traffic_from_profile()
    log(f"{DOMINANT_KERNEL}: {kern_us:.2f} us/launch")

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
            "workload": "RWKV7-0.4B decode B=1 (config 3): one persistent kernel launch per token",
            "layers": shape.n_layer,
            "n_embd": shape.n_embd,
            "vocab": V,
            "batch": 1,
        },
        "tokens_per_s": round(1000.0 / ms_tok, 1),
        "correctness": gate,
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
    out["roofline"] = {
        "bound": "hbm",
        "achieved": round(kern_gbs, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(kern_gbs / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "kernel": DOMINANT_KERNEL,
        "avg_launch_us": round(kern_us, 2),
        "alg_bytes_per_launch": step_bytes,
    }

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
        # ---- decode B=1 on int8 weights (the same persistent kernel streaming
        # per-row int8 matrices and head, f32 row scales) ----
        model8 = RWKV7HIP(w, is_torch_compile=False, weight_quant="int8")
        S8 = State(w.L, w.C, 64, device=dev)
        for i in range(Wm):
            model8.decode_into(toks[i], S8, logits1)
        us_i8 = time_cuda(lambda it=iter(range(K)): model8.decode_into(toks[next(it) % (K + Wm)], S8, logits1),
                          min(K, 128)) * 1e3
        i8_bytes = int8_decode_bytes(shape, step_bytes)
        out["decode_int8"] = {
            "us_per_token": round(us_i8, 2),
            "alg_bytes": i8_bytes,
            "hbm_frac": round(i8_bytes / (us_i8 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        }
        log(f"decode B=1 int8 weights: {us_i8:.2f} us/token")
        del model8, S8
        # ---- decode B=1 of the bfloat16 model (same seed, bf16 weights) ----
        from rwkv_tl_amd import RWKV7HIPBF16

        sdb = make_random_state_dict("0.4b", seed=0, dtype=torch.bfloat16)
        wb = RWKV7Weight.from_state_dict(sdb, device=dev, dtype=torch.bfloat16)
        del sdb
        modelb = RWKV7HIPBF16(wb, is_torch_compile=False)
        Sb = modelb.new_state()
        logitsb = torch.empty(1, V, dtype=torch.bfloat16, device=dev)
        for i in range(Wm):
            modelb.decode_into(toks[i], Sb, logitsb)
        us_bf = time_cuda(lambda it=iter(range(K)): modelb.decode_into(toks[next(it) % (K + Wm)], Sb, logitsb),
                          min(K, 128)) * 1e3
        out["decode_bf16"] = {
            "us_per_token": round(us_bf, 2),
            "hbm_frac": round(step_bytes / (us_bf * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        }
        log(f"decode B=1 bf16 model: {us_bf:.2f} us/token")
        del modelb, Sb, wb
        # ---- int8 weight-only GEMV vs the f16 GEMV on the head shape ----
        # (direct C-ABI calls into a preallocated output, so the host wrapper's
        # checks and allocation stay out of the timed launches)
        from rwkv_tl_amd import _lib as LB
        from rwkv_tl_amd import kernels as KO

        Wh = w.head.contiguous()
        Nh = Wh.shape[0]
        qh, sh = KO.quantize_i8(Wh)
        xh = torch.randn(w.C, generator=g).to(dev)
        yh = torch.empty(Nh, dtype=torch.float32, device=dev)
        lib, sth = LB.load(), LB.stream_handle()
        g8 = lambda: lib.rwkv7_gemv_i8(xh.data_ptr(), qh.data_ptr(), w.C, sh.data_ptr(), yh.data_ptr(), Nh, w.C, sth)
        g16 = lambda: lib.rwkv7_gemv_f16(xh.data_ptr(), Wh.data_ptr(), w.C, yh.data_ptr(), Nh, w.C, 0, sth)
        LB.check(g8(), "rwkv7_gemv_i8")
        LB.check(g16(), "rwkv7_gemv_f16")
        us8 = time_cuda(g8, 100) * 1e3
        us16 = time_cuda(g16, 100) * 1e3
        c4, l4 = KO.quantize_any4(Wh)
        g4 = lambda: lib.rwkv7_gemv_any4(xh.data_ptr(), c4.data_ptr(), c4.stride(0), l4.data_ptr(), yh.data_ptr(),
                                         Nh, w.C, sth)
        LB.check(g4(), "rwkv7_gemv_any4")
        us4 = time_cuda(g4, 100) * 1e3
        b8, b16h = Nh * w.C + 8 * Nh + 4 * w.C, 2 * Nh * w.C + 4 * Nh + 4 * w.C
        b4 = Nh * w.C // 2 + 32 * Nh + 4 * Nh + 4 * w.C
        out["gemv_i8_head"] = {
            "shape": [Nh, w.C],
            "i8_us": round(us8, 2),
            "i8_hbm_frac": round(b8 / (us8 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "f16_us": round(us16, 2),
            "f16_hbm_frac": round(b16h / (us16 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "any4_us": round(us4, 2),
            "any4_hbm_frac": round(b4 / (us4 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        }
        log(f"gemv head {Nh}x{w.C}: int8 {us8:.2f} us, any4 {us4:.2f} us, f16 {us16:.2f} us")
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
        for k, v in pre.items():
            out[f"prefill_{k}_ms"] = v["ms"]
            out[f"prefill_{k}_hbm_frac"] = v["hbm_frac"]
            out[f"prefill_{k}_mfma_frac"] = v["mfma_frac"]
            out[f"prefill_{k}_tokens_per_s"] = v["tokens_per_s"]

    if args.calib_copy:
        calib_copy()
    if not args.no_cpu:
        log(f"CPU baseline: {args.cpu_steps} decode steps and a 1x128 prefill of the fp32 oracle")
        out["cpu_baseline"] = cpu_baseline(ref_w, args.cpu_steps, 1, 128)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
