"""Benchmark of the YufMusicGen recurrent hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

One "step" is the C3 prefill of BASELINE.json: the default 0.1B model
(14 layers, d_model 640, 16 heads x 40, ROSA 128, vocab 20 480, random fp32
weights from a seed) over B = 8 rows x T = 2048 synthetic token ids, every
position's logits written to HBM.  Token ids and weights are resident in HBM
before the timed region; W untimed steps, then exactly K timed steps between
device synchronisations.  `value` = B*T*K / elapsed (prefill tokens/s).

In the same run:
  * decode (C4): 64 streams prefilled with 256 tokens, then 1024 single-token
    steps with on-device temperature-1.0 top-k=32 sampling -> decode tokens/s;
  * the WKV-7 scan (C2: B=8, T=2048, H=16, N=40, zero state) timed with HIP
    events on the stream it runs on -> `roofline` (algorithmic bytes / time
    against the 8 TB/s HBM peak);
  * `decode_roofline`: the whole C4 decode step's algorithmic bytes (646.5 MB:
    weights, state read and written, logits) over its measured time, against
    8 TB/s, with the operator-form single-token WKV-7 step kernel timed alone
    beside it; the ROSA scan of a C3 layer -> `rosa_roofline`;
  * `c5`: C5 as configured with bf16 weights -- the wide model (24 layers,
    d_model 1024, 16 x 64 heads, ROSA 256), B = 32 x T = 8192 prefill in
    T-chunks of 2048 (last-position logits), then 512 decode steps of the 32
    streams with device top-k sampling (--no-c5 skips it);
  * the FFN in/gate projection GEMM of C3 (M=16384, N=5120, K=640) -> MFMA
    utilisation: fp32 products run as six bf16 MFMAs over three-part bf16
    splits, so the peak is the 2.5 PFLOP/s dense bf16 peak / 6 (416.7 TFLOP/s
    fp32-equivalent; YUF_GEMM_X3=0 measures the fp32 MFMA form against the
    157.3 TFLOP/s fp32 peak);
  * `cpu_baseline`: the oracle's float32 restatement of the reference's PyTorch
    CPU fallback on a bounded slice of C3 (same model, B=8 x T=1024), timed on
    this host's cores (~10-30 s of CPU work).

Only N = 1 GPU exists on these boxes; --gpus above 1 exits with a message.

`--only c5`: the C5 leg alone, and the same workload with fp32 weights.

`cpu_baseline_decode` / `cpu_baseline_scan`: the oracle's float32 single-token
step of C4 (64 streams) and its sequential C2 scan, on the same host cores.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "prefill+decode tokens/s, 0.1B model B=8 T=2048; WKV-7 scan % of HBM roofline"
HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2500.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def wkv_bytes(B, T, H, N, nonzero_state=False) -> int:
    """Algorithmic HBM bytes of one scan: r, w, k, v, a, b in, y out, final state out (+ state in)."""
    return 4 * (7 * B * T * H * N + B * H * N * N * (2 if nonzero_state else 1))


def time_events(fn, iters: int, stream=None) -> float:
    """Average ms per call, HIP events recorded on `stream` (a torch.cuda.Stream)."""
    import torch

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters


def bench_scan(iters: int) -> dict:
    import torch

    from yufmusicgen_amd.ops import rwkv7_scan
    from yufmusicgen_amd.synth import wkv_inputs

    B, T, H, N = 8, 2048, 16, 40
    dev = [torch.from_numpy(x).cuda() for x in wkv_inputs(0, B, T, H, N)]
    rwkv7_scan(*dev)
    torch.cuda.synchronize()
    ms = time_events(lambda: rwkv7_scan(*dev), iters, torch.cuda.current_stream())
    nbytes = wkv_bytes(B, T, H, N)
    achieved = nbytes / (ms * 1e-3) / 1e9
    traffic = None
    pmc = os.path.join(ROOT, "profiles", "wkv7_scan_c2_traffic.json")
    if os.path.exists(pmc):
        with open(pmc) as handle:
            traffic = json.load(handle).get("traffic_bytes")
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": "wkv7_chunk_kernel<3,false,true,true> (C2: B=8 T=2048 H=16 N=40; two workgroups per head, half-padded last key tile)",
            "algorithmic_bytes": nbytes, "avg_us": round(ms * 1e3, 2)}


def decode_step_bytes(cfg, streams: int) -> int:
    """Algorithmic HBM bytes of one decode step: every
    weight once (the tied embedding once, as the LM head; the gathered rows are
    negligible), each stream's recurrent state read and written (previous, WKV,
    ROSA), and the V logits written.  0.1B model, 64 streams: 646.5 MB."""
    from yufmusicgen_amd.synth import tensor_specs

    params = sum(int(np.prod(shape)) for _, shape in tensor_specs(cfg))
    state = cfg.n_layers * (cfg.d_model + cfg.n_heads * cfg.head_size ** 2 + cfg.rosa_size)
    return 4 * (params + 2 * streams * state + streams * cfg.vocab_size)


def wkv_step_in_model_bytes(cfg, n: int) -> int:
    """Algorithmic bytes of one in-model WKV-7 step launch (the fused form
    with the second low-rank stage) for n streams: per stream the state read
    and written (8 B x H N^2), r, k, v and the three rank-L rows read, y and
    the output gate written; once per launch w2t / a2t / g2t ([d, L] each)
    and w0, a0, k_k, k_a ([d] each)."""
    d, L, hn2 = cfg.d_model, cfg.low_rank, cfg.n_heads * cfg.head_size ** 2
    per_stream = 8 * hn2 + 12 * d + 12 * L + 8 * d
    return n * per_stream + 12 * d * L + 16 * d


def wkv_step_in_model(engine, cfg, iters: int = 50) -> dict:
    """The decode step's own WKV-7 kernel (wkv7_step_kernel<N,true,4,true>,
    low-rank stage folded in, the first layer of the last step's stream
    group), relaunched alone with its inputs from a replayed HIP graph and
    timed with HIP events on the engine's stream (yuf_engine_time_wkv_step);
    the time per launch includes the graph's dispatch gap between kernels."""
    us, n = engine.time_wkv_step(iters)
    nbytes = wkv_step_in_model_bytes(cfg, n)
    achieved = nbytes / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "avg_us": round(us, 2), "streams": n,
            "algorithmic_bytes": nbytes,
            "kernel": f"wkv7_step_kernel<{cfg.head_size},true,4,true> (in-model, {n} streams, low-rank stage folded in)"}


def decode_roofline(cfg, streams: int, ms_per_step: float, operator_leg: dict, in_model: dict = None) -> dict:
    """The whole decode step against the HBM roofline: algorithmic bytes per
    step / measured step time (the step is a chain of dependent launches, so
    this is the figure to move); beside it the step's own WKV-7 kernel timed
    alone (in_model) and the operator-form WKV-7 step kernel
    (wkv7_step_kernel<N,false,1,false> through yuf_wkv7_scan_f32)."""
    nbytes = decode_step_bytes(cfg, streams)
    achieved = nbytes / (ms_per_step * 1e-3) / 1e9
    traffic = None
    pmc = os.path.join(ROOT, "profiles", "decode_c4_traffic.json")
    if os.path.exists(pmc):
        with open(pmc) as handle:
            traffic = json.load(handle).get("step", {}).get("traffic_bytes")
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": f"whole C4 decode step ({streams} streams, 0.1B model, graph-replayed)",
            "algorithmic_bytes": nbytes, "ms_per_step": round(ms_per_step, 4), "wkv_step_in_model": in_model,
            "wkv_step_operator": operator_leg}


def bench_wkv_step(iters: int) -> dict:
    """The single-token WKV-7 step of C4 (64 streams, H=16, N=40, state read and
    written in place): 64 (2 H N^2 + 7 d) 4 bytes = 14.25 MB per layer-step."""
    import torch

    from yufmusicgen_amd._lib import check, lib
    from yufmusicgen_amd.synth import wkv_inputs

    B, H, N = 64, 16, 40
    dev = [torch.from_numpy(x).cuda() for x in wkv_inputs(2, B, 1, H, N)]
    y = torch.empty_like(dev[0])
    state = torch.randn(B, H, N, N, device="cuda") * 0.1
    st = torch.cuda.current_stream().cuda_stream
    run = lambda: check(lib().yuf_wkv7_scan_f32(B, 1, H, N, *[x.data_ptr() for x in dev],  # noqa: E731
                                                state.data_ptr(), state.data_ptr(), y.data_ptr(), st))
    run()
    torch.cuda.synchronize()
    ms = time_events(run, iters, torch.cuda.current_stream())
    nbytes = B * (2 * H * N * N + 7 * H * N) * 4
    achieved = nbytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "kernel": "wkv7_step_kernel<40,false,1,false> operator form (C4: 64 streams, H=16, N=40, T=1)",
            "algorithmic_bytes": nbytes, "avg_us": round(ms * 1e3, 2)}


def bench_rosa(iters: int) -> dict:
    """ROSA scan of one C3 layer (B=8, T=2048, D=128, gated read) through the
    operator entry point (segmented form: A^64 on the device, segments from
    zero, carry chain, segments again): 4 (4 B T D + 2 B D) bytes = 33.6 MB."""
    import torch

    from yufmusicgen_amd._lib import check, lib
    from yufmusicgen_amd.synth import rosa_inputs

    B, T, D = 8, 2048, 128
    cand, write, read_raw, decay, u = [torch.from_numpy(x).cuda() for x in rosa_inputs(4, B, T, D)]
    mem = torch.zeros(B, D, device="cuda")
    out = torch.empty(B, T, D, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    run = lambda: check(lib().yuf_rosa_scan_f32(B, T, D, cand.data_ptr(), write.data_ptr(),  # noqa: E731
                                                read_raw.data_ptr(), decay.data_ptr(), u.data_ptr(),
                                                mem.data_ptr(), mem.data_ptr(), out.data_ptr(), st))
    run()
    torch.cuda.synchronize()
    ms = time_events(run, iters, torch.cuda.current_stream())
    nbytes = 4 * (4 * B * T * D + 2 * B * D)
    achieved = nbytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "kernel": "rosa operator, segmented (rosa_power/scan/carry/scan; C3 layer: B=8 T=2048 D=128)",
            "algorithmic_bytes": nbytes, "avg_us": round(ms * 1e3, 2)}


def bench_gemm(iters: int) -> dict:
    import torch

    from yufmusicgen_amd._lib import check, lib

    M, N, K = 16384, 5120, 640
    a = torch.randn(M, K, device="cuda")
    w = torch.randn(N, K, device="cuda") * 0.02
    c = torch.empty(M, N, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    # W pre-split once into its three bf16 parts, as the engine does for every
    # projection matrix at creation (not timed).
    planes = torch.empty(lib().yuf_x3_planes_elems(N, K), dtype=torch.int16, device="cuda")
    check(lib().yuf_x3_split_planes(N, K, w.data_ptr(), planes.data_ptr(), st))
    run = lambda: check(lib().yuf_linear_f32_planes(M, N, K, a.data_ptr(), w.data_ptr(),  # noqa: E731
                                                    planes.data_ptr(), None, 0, None, c.data_ptr(), st))
    for _ in range(5):  # untimed: the first launches run at lower clocks
        run()
    torch.cuda.synchronize()
    ms = time_events(run, iters, torch.cuda.current_stream())
    tflops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    if os.environ.get("YUF_GEMM_X3", "1") == "0":
        return {"bound": "mfma", "achieved": round(tflops, 2), "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tflops / FP32_MFMA_PEAK_TFLOPS, 4),
                "kernel": "gemm_big_kernel<256,true> fp32 MFMA, M=16384 N=5120 K=640", "avg_us": round(ms * 1e3, 1)}
    # fp32 products as six bf16 MFMAs over three-part splits: the fp32-equivalent
    # peak of that form is the bf16 dense peak / 6.
    peak = BF16_MFMA_PEAK_TFLOPS / 6.0
    return {"bound": "mfma", "achieved": round(tflops, 2), "peak": round(peak, 1), "unit": "TFLOP/s",
            "frac": round(tflops / peak, 4), "fp32_mfma_peak": FP32_MFMA_PEAK_TFLOPS,
            "kernel": "gemm_x3p_kernel<256,true,4> (fp32 via 6 bf16 MFMAs, pre-split W planes, 256-row tiles), M=16384 N=5120 K=640",
            "avg_us": round(ms * 1e3, 1)}


def bench_c5(args, weight_types=("bf16", "f32")) -> dict:
    """C5 as configured: the wide model (24 layers,
    d_model 1024, 16 x 64 heads, ROSA 256, V 20480) with bf16 projection weights
    and fp32 WKV / ROSA state; B = 32 rows x T = 8192 tokens of prefill
    (T-chunked through a 32 x 2048-token engine pass, the state carried,
    last-position logits), then 512 decode steps of the 32 streams with device
    top-k = 32, T = 1.0 sampling.  The fp32-weight engine runs the same workload
    once for comparison (--only c5; the default run measures bf16 only)."""
    import torch

    from yufmusicgen_amd.checkpoint import write_yuf
    from yufmusicgen_amd.config import PRESETS
    from yufmusicgen_amd.engine import Checkpoint, Engine, sample_device
    from yufmusicgen_amd.synth import prompt_tokens, synth_weights

    cfg = PRESETS["wide"]
    log("c5: generating weights")
    weights = synth_weights(cfg, seed=0)
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "c5.yuf")
        write_yuf(path, cfg, weights, linear_bf16=True)
        ckpt = Checkpoint.load(path)
    del weights
    B, T, D, chunk = 32, 8192, args.c5_decode_steps, 2048
    tokens = torch.from_numpy(prompt_tokens(0, B, T, cfg.vocab_size)).cuda()
    slots = np.arange(B, dtype=np.int32)
    out = {"workload": f"C5: 24L d=1024 16x64 ROSA 256 V=20480, bf16 weights (.yuf v2), prefill {B}x{T} "
                       f"(T-chunks of {chunk}, last logits), then {D} decode steps of {B} streams "
                       "(device top-k=32 T=1.0 sampling)"}
    for wt, reps in (("bf16", max(1, args.c5_steps)), ("f32", 1)):
        if wt not in weight_types:
            continue
        engine = Engine(ckpt, max_streams=B, max_tokens=B * chunk, weight_dtype=wt)
        stream = torch.cuda.ExternalStream(engine.stream)
        logits = torch.empty(B, cfg.vocab_size, device="cuda")
        step_tok = torch.empty(B, dtype=torch.int32, device="cuda")  # one buffer: the step graph reads it in place
        engine.reset_state()
        engine.prefill_device(tokens, logits, slots, logits="last")  # warm-up (capture, first touches)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            engine.reset_state()
            engine.prefill_device(tokens, logits, slots, logits="last")
        torch.cuda.synchronize()
        pf = (time.perf_counter() - t0) / reps
        with torch.cuda.stream(stream):
            sample_device(logits, step_tok, 1.0, 32, seed=99, counter=0, stream=engine.stream)
        for i in range(3):  # warm-up steps (graph capture)
            engine.step_device(step_tok, logits, slots)
            sample_device(logits, step_tok, 1.0, 32, seed=99, counter=1 + i, stream=engine.stream)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(D):
            engine.step_device(step_tok, logits, slots)
            sample_device(logits, step_tok, 1.0, 32, seed=99, counter=100 + i, stream=engine.stream)
        torch.cuda.synchronize()
        dc = (time.perf_counter() - t0) / D
        engine.take_error()
        out[wt] = {"prefill_tokens_per_s": round(B * T / pf), "prefill_ms": round(pf * 1e3, 2),
                   "decode_tokens_per_s": round(B / dc), "decode_ms_per_step": round(dc * 1e3, 3),
                   "prefill_reps": reps}
        log(f"c5 {wt}: prefill {pf * 1e3:.1f} ms ({B * T / pf:.0f} tok/s), decode {dc * 1e3:.3f} ms/step")
        engine.close()
        del engine
        torch.cuda.empty_cache()
    return out


def _cpu_threads() -> int:
    import torch

    torch.set_num_threads(max(1, len(os.sched_getaffinity(0))))
    return torch.get_num_threads()


def cpu_baseline(weights, cfg) -> dict:
    import torch

    from oracle.model import OracleModel
    from yufmusicgen_amd.synth import prompt_tokens

    cores = _cpu_threads()
    B, T = 8, 1024
    tokens = prompt_tokens(7, B, T, cfg.vocab_size)
    model = OracleModel(cfg.to_dict(), weights, dtype=torch.float32)
    with torch.no_grad():
        model.forward(tokens[:, :4])  # warm-up
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            model.forward(tokens, logits="all")
            times.append(time.perf_counter() - t0)
    sec = float(np.median(times))
    return {"value": round(B * T / sec, 2), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"C3 prefill slice B={B} x T={T} (0.1B model, all-position logits), fp32 torch CPU "
                      f"restatement of the reference fallback, median of 3 = {sec:.2f} s"}


def cpu_baseline_decode(weights, cfg, steps: int = 8) -> dict:
    """C4 decode on the host: the float32 oracle's single-token step
    (model.py:424-431, the per-token path of cli/generate.py:139-154) for 64
    streams from a 256-token prefilled state, median of `steps` steps."""
    import torch

    from oracle.model import OracleModel
    from yufmusicgen_amd.synth import uniform_tokens

    cores = _cpu_threads()
    S, P = 64, 256
    model = OracleModel(cfg.to_dict(), weights, dtype=torch.float32)
    with torch.no_grad():
        _, state = model.forward(uniform_tokens(3, S, P, cfg.vocab_size), logits="last")
        nxt = uniform_tokens(4, S, steps + 1, cfg.vocab_size)
        _, state = model.step(nxt[:, 0], state)  # warm-up
        times = []
        for t in range(1, steps + 1):
            t0 = time.perf_counter()
            _, state = model.step(nxt[:, t], state)
            times.append(time.perf_counter() - t0)
    sec = float(np.median(times))
    return {"value": round(S / sec, 2), "unit": "tokens/s", "cores": cores, "kind": "port",
            "ms_per_step": round(sec * 1e3, 2),
            "sample": f"C4 decode: {steps} single-token steps of {S} streams after a {P}-token prefill (0.1B model), "
                      f"fp32 torch CPU restatement of the reference's per-token path, median step {sec * 1e3:.1f} ms"}


def cpu_baseline_scan() -> dict:
    """C2 on the host: the float32 oracle's sequential WKV-7 scan
    (model.py:145-165) at the full C2 shape, median of 3."""
    import torch

    from oracle import wkv7 as owkv
    from yufmusicgen_amd.synth import wkv_inputs

    cores = _cpu_threads()
    B, T, H, N = 8, 2048, 16, 40
    arrs = [torch.from_numpy(x) for x in wkv_inputs(0, B, T, H, N)]
    with torch.no_grad():
        owkv.wkv7_scan(*(x[:, :16] for x in arrs))  # warm-up
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            owkv.wkv7_scan(*arrs)
            times.append(time.perf_counter() - t0)
    sec = float(np.median(times))
    nbytes = wkv_bytes(B, T, H, N)
    return {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s (algorithmic)", "cores": cores, "kind": "port",
            "us_per_scan": round(sec * 1e6, 1), "tokens_per_s": round(B * T / sec, 1),
            "sample": f"C2 scan B={B} T={T} H={H} N={N}, zero state, fp32 torch CPU restatement of the "
                      f"reference recurrence, median of 3 = {sec:.3f} s"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--decode-steps", type=int, default=1024)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--c5-steps", type=int, default=2, help="timed C5 prefills")
    ap.add_argument("--c5-decode-steps", type=int, default=512, help="C5 decode steps")
    ap.add_argument("--no-c5", action="store_true", help="skip the C5 leg of the default run")
    ap.add_argument("--only", choices=["scan", "prefill", "decode", "copy", "c5", "kernels", "gemm"], default=None,
                    help="profiling aids: just the C2 scan (20 launches), just the prefill steps, just the C4 "
                         "decode leg, a plain 256 MiB device copy (20 launches) that calibrates the "
                         "FETCH_SIZE/WRITE_SIZE counters, the three HBM-bound kernel legs, or the FFN "
                         "projection GEMM alone (11 launches)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path would shard data-parallel over streams: one engine per GPU, each "
              "holding its own streams' recurrent state)", file=sys.stderr)
        return 2

    import torch

    if args.only == "scan":
        print(json.dumps({"roofline": bench_scan(20)}), flush=True)
        return 0
    if args.only == "kernels":  # the three HBM-bound kernel legs, for one profiling run
        print(json.dumps({"roofline": bench_scan(20), "decode_roofline": bench_wkv_step(50),
                          "rosa_roofline": bench_rosa(20)}), flush=True)
        return 0
    if args.only == "gemm":
        print(json.dumps({"gemm_roofline": bench_gemm(10)}), flush=True)
        return 0
    if args.only == "copy":
        src = torch.ones(64 << 20, device="cuda")
        dst = torch.empty_like(src)
        ms = time_events(lambda: dst.copy_(src), 20, torch.cuda.current_stream())
        print(json.dumps({"copy_bytes_each_way": src.numel() * 4, "avg_us": round(ms * 1e3, 2)}), flush=True)
        return 0

    from yufmusicgen_amd.checkpoint import write_yuf
    from yufmusicgen_amd.config import PRESETS
    from yufmusicgen_amd.engine import Checkpoint, Engine, sample_device
    from yufmusicgen_amd.synth import prompt_tokens, synth_weights, uniform_tokens

    if args.only == "c5":
        print(json.dumps({"c5": bench_c5(args)}), flush=True)
        return 0

    cfg = PRESETS["0.1b"]
    log("generating weights")
    weights = synth_weights(cfg, seed=0)
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "model.yuf")
        write_yuf(path, cfg, weights)
        ckpt = Checkpoint.load(path)
    B, T = 8, 2048
    engine = Engine(ckpt, max_streams=64, max_tokens=B * T)
    stream = torch.cuda.ExternalStream(engine.stream)
    tokens = torch.from_numpy(prompt_tokens(0, B, T, cfg.vocab_size)).cuda()
    logits = torch.empty(B, T, cfg.vocab_size, device="cuda")
    slots = np.arange(B, dtype=np.int32)

    def prefill_step():
        engine.prefill_device(tokens, logits, slots, logits="all")

    ms_per_step = prefill_tps = None
    if args.only != "decode":
        log("prefill warmup")
        for _ in range(args.warmup):
            engine.reset_state()
            prefill_step()
        torch.cuda.synchronize()
        log("prefill timed")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            prefill_step()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        ms_per_step = elapsed * 1e3 / args.steps
        prefill_tps = B * T * args.steps / elapsed
        log(f"prefill {ms_per_step:.2f} ms/step, {prefill_tps:.0f} tokens/s")
    if args.only == "prefill":
        print(json.dumps({"prefill_tokens_per_s": prefill_tps, "ms_per_step": ms_per_step}), flush=True)
        return 0

    # C4 decode: 64 streams x 256-token prefill, then decode with device top-k sampling.
    S, P = 64, 256
    engine.reset_state()
    dec_tokens = torch.from_numpy(uniform_tokens(3, S, P, cfg.vocab_size)).cuda()
    last_logits = torch.empty(S, cfg.vocab_size, device="cuda")
    dslots = np.arange(S, dtype=np.int32)
    engine.prefill_device(dec_tokens, last_logits, dslots, logits="last")
    step_tok = torch.empty(S, dtype=torch.int32, device="cuda")
    with torch.cuda.stream(stream):
        sample_device(last_logits, step_tok, 1.0, 32, seed=1234, counter=0, stream=engine.stream)
    for i in range(3):  # warm-up steps
        engine.step_device(step_tok, last_logits, dslots)
        sample_device(last_logits, step_tok, 1.0, 32, seed=1234, counter=i + 1, stream=engine.stream)
    torch.cuda.synchronize()
    log("decode timed")
    t0 = time.perf_counter()
    for i in range(args.decode_steps):
        engine.step_device(step_tok, last_logits, dslots)
        sample_device(last_logits, step_tok, 1.0, 32, seed=1234, counter=100 + i, stream=engine.stream)
    torch.cuda.synchronize()
    dec_elapsed = time.perf_counter() - t0
    decode_tps = S * args.decode_steps / dec_elapsed
    log(f"decode {dec_elapsed * 1e3 / args.decode_steps:.3f} ms/step, {decode_tps:.0f} tokens/s")
    wkv_in_model = wkv_step_in_model(engine, cfg)
    log(f"in-model WKV step {wkv_in_model['avg_us']} us ({wkv_in_model['frac']:.3f} of HBM)")
    if args.only == "decode":
        print(json.dumps({"decode_tokens_per_s": decode_tps, "decode_ms_per_step": dec_elapsed * 1e3 / args.decode_steps,
                          "wkv_step_in_model": wkv_in_model}), flush=True)
        return 0
    engine.close()
    del logits

    c5 = None
    if not args.no_c5:
        del engine
        torch.cuda.empty_cache()
        log("c5 (bf16 weights)")
        c5 = bench_c5(args, weight_types=("bf16",))
    log("scan roofline")
    roofline = bench_scan(20)
    log(f"scan {roofline['avg_us']} us, {roofline['achieved']} GB/s")
    step = bench_wkv_step(50)
    log(f"wkv step {step['avg_us']} us, {step['achieved']} GB/s")
    rosa = bench_rosa(20)
    log(f"rosa {rosa['avg_us']} us, {rosa['achieved']} GB/s")
    gemm = bench_gemm(10)
    log(f"gemm {gemm['achieved']} TFLOP/s")
    cpu = cpu_dec = cpu_scan = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        cpu = cpu_baseline(weights, cfg)
        log(f"cpu {cpu['value']} tokens/s on {cpu['cores']} cores")
        cpu_dec = cpu_baseline_decode(weights, cfg)
        log(f"cpu decode {cpu_dec['value']} tokens/s ({cpu_dec['ms_per_step']} ms/step)")
        cpu_scan = cpu_baseline_scan()
        log(f"cpu scan {cpu_scan['us_per_scan']} us ({cpu_scan['value']} GB/s)")

    out = {
        "metric": METRIC,
        "value": round(prefill_tps, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "C3 prefill: 0.1B model (14L, d640, 16x40 heads, ROSA 128, V 20480, seeded fp32 weights), "
                        "B=8 x T=2048 token ids, all-position logits",
            "prefill_streams": os.environ.get("YUF_PREFILL_GROUPS", "4 (automatic: the batch's 128 heads as four "
                                                                    "parts of two sequences)"),
            "decode_workload": f"C4: 64 streams prefilled with 256 tokens, {args.decode_steps} steps, "
                               "device top-k=32 T=1.0 sampling",
            "decode_streams": os.environ.get("YUF_DECODE_BRANCHES", "2 (automatic: two 32-stream step graphs)"),
        },
        "decode_tokens_per_s": round(decode_tps, 1),
        "decode_ms_per_step": round(dec_elapsed * 1e3 / args.decode_steps, 3),
        "roofline": roofline,
        "decode_roofline": decode_roofline(cfg, S, dec_elapsed * 1e3 / args.decode_steps, step, wkv_in_model),
        "rosa_roofline": rosa,
        "gemm_roofline": gemm,
        "cpu_baseline": cpu,
        "cpu_baseline_decode": cpu_dec,
        "cpu_baseline_scan": cpu_scan,
        "c5": c5,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
