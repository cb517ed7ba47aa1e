#!/usr/bin/env python3
"""Benchmark of the brisk-llm token loop on one MI355X.

Workload: the Qwen3-0.6B-shaped decoder, Q4_0 layers with
Q8_0 embeddings and output, random weights from a seeded GGUF; 32 random prompt
ids, then greedy decode.  A "step" is one decode token: the full forward pass
(28 layers + output projection + on-device greedy pick).  All K timed steps run
in one launch of the persistent token loop (k_loop); inputs (weights, KV cache,
token sequence) are resident in HBM when the timed region starts.

Printed (one JSON line): decode tok/s as `value`, plus
  roofline      the dominant kernel, k_loop (one launch = the K decode steps),
                timed with HIP events on the session's stream: algorithmic
                bytes of the K steps (weights + norms + KV read/write per token)
                over the launch time, against MI355X's 8 TB/s HBM peak;
  q4_0_gemv     configs[0]'s 2048 x 2048 Q4_0 matvec (k_gemv): single-launch
                latency, and streaming GB/s over 128 distinct copies (302 MB,
                beyond the 256 MB Infinity Cache);
  output_gemv   the 151936 x 1024 Q8_0 output projection as one k_gemv launch;
  prefill       tok/s of a 512-token prompt on the Llama-3.2-1B Q4_K_M shape;
  cpu_baseline  the reference's own CPU engine (built from its sources with its
                portable kernels, oracle/_ref) on this host, on the same decode
                workload (32-id prompt, 256 greedy tokens).
`--copy-calibration MB` instead runs one device-to-device copy of that size (the
plain copy kernel the rocprofv3 FETCH_SIZE/WRITE_SIZE readings are scaled by).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "brisk-llm_amd"), os.path.join(ROOT, "oracle")]

HBM_PEAK = 8.0e12


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_events(torch, stream_ptr, fn, reps):
    """Average ms of fn() over reps, with HIP events recorded on the given stream."""
    st = torch.cuda.ExternalStream(stream_ptr) if stream_ptr else torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(st)
    for i in range(reps):
        fn(i)
    end.record(st)
    end.synchronize()
    return start.elapsed_time(end) / reps


def gemv_roofline(torch, lib, L, rows, cols, ttype, block_bytes, copies, reps, norm, graph=False):
    """Streams the GEMV over `copies` distinct packed matrices; returns (ms per launch, bytes per launch), and with
    `graph` also the ms per launch of the same launches replayed from a HIP graph."""
    import ctypes as C
    import numpy as np
    from brisk_hip import synth
    be = 32 if ttype in (2, 8) else 256
    nb = rows * cols // be
    raw = synth.BLOCK_MAKERS[ttype](12345, nb).reshape(-1)
    src = torch.from_numpy(raw.copy()).cuda()
    nbytes = lib.brisk_hip_packed_bytes(ttype, rows, cols)
    mats = []
    for _ in range(copies):
        d = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        L.check(lib.brisk_hip_pack(ttype, C.c_void_p(src.data_ptr()), rows, cols, C.c_void_p(d.data_ptr()), None))
        mats.append(d)
    del src
    x = torch.randn(cols, device="cuda")
    w = torch.ones(cols, device="cuda") if norm else None
    out = torch.empty(rows, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def launch(i, st=stream):
        L.check(lib.brisk_hip_gemv(ttype, 0, C.c_void_p(mats[i % copies].data_ptr()), rows, cols, C.c_void_p(x.data_ptr()),
                                   C.c_void_p(w.data_ptr()) if w is not None else None, 1e-6, C.c_void_p(out.data_ptr()), 0,
                                   C.c_void_p(st)))

    for i in range(copies):
        launch(i)
    torch.cuda.synchronize()
    ms = time_events(torch, stream, launch, reps)
    # the same launches replayed from a HIP graph: the device time a launch takes, without the
    # host's per-call cost (the eager loop above is bound by the ctypes call at these sizes)
    ms_graph = None
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            cap = torch.cuda.current_stream().cuda_stream
            for i in range(reps):
                launch(i, cap)
        g.replay()
        torch.cuda.synchronize()
        ms_graph = time_events(torch, 0, lambda i: g.replay(), 4) / reps
        del g
    algo = rows * cols // be * block_bytes + cols * 4 * (2 if norm else 1) + rows * 4
    del mats
    torch.cuda.empty_cache()
    return (ms, algo, ms_graph) if graph else (ms, algo)


def cpu_baseline(path, prompt, n_gen):
    import pyoracle
    if not pyoracle.ref_available():
        return None
    # `-t $(nproc)` as BASELINE.md runs the reference: nproc counts the cores this process may run on
    nproc = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    threads = max(1, min(128, nproc))
    ref = pyoracle.Reference(path, threads=threads, max_context=len(prompt) + n_gen + 8)
    ids, gaps, pre_s, gen_s = ref.generate(prompt, n_gen)
    ref.close()
    one = pyoracle.Reference(path, threads=1, max_context=len(prompt) + 16)
    _, _, pre1, gen1 = one.generate(prompt, 8)
    one.close()
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    return {"value": round((n_gen - 1) / gen_s, 3), "unit": "tok/s", "cores": threads, "kind": "reference",
            "sample": f"the full decode workload: qwen3-0.6b-shape, {len(prompt)}-id prompt then {n_gen} greedy tokens "
                      f"(generation tok/s = (tokens - 1) / generation seconds, as src/main.cpp:312-318; {threads} threads "
                      f"of {model or 'host CPU'}); prompt {len(prompt) / pre_s:.1f} tok/s",
            "one_thread_tok_s": round(7 / gen1, 3), "nproc": nproc, "cpu_count": os.cpu_count(),
            "ids": ids}


def other_configs(torch, HipSession, model, synth):
    """configs[3] (Qwen3-1.7B Q8_0, KV pre-filled to 4096 with fp16 N(0,1), 128 decode steps) and
    configs[4] (BitNet-2B TQ2_0, 64-id prompt, 256 greedy steps): decode tok/s."""
    import ctypes as C
    import numpy as np
    out = {}
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    f, cfg, table = model.load(synth.model_path("qwen3-1.7b"))
    gguf_bytes = sum(t.data.nbytes for t in table)
    for t in table:                    # the file's pages resident, as after the reference's mmap + first touch
        int(np.asarray(t.data[::4096], dtype=np.uint64).sum())
    load = {}
    for mode in ("pageable", "pinned"):  # session creation: upload + repack of every tensor
        if mode == "pageable":
            os.environ["BRISK_HIP_PAGEABLE_UPLOAD"] = "1"
        t0 = time.perf_counter()
        s = HipSession((f, cfg, table), max_context=4096 + 160)
        torch.cuda.synchronize()
        load[mode] = time.perf_counter() - t0
        os.environ.pop("BRISK_HIP_PAGEABLE_UPLOAD", None)
        if mode == "pageable":
            s.close()
            del s
    out["load_qwen3-1.7b"] = {"workload": "session creation of configs[3] (upload of the GGUF bytes, repack to planes, "
                                          "caches for 4256 positions)", "gguf_bytes": gguf_bytes,
                              "seconds": round(load["pinned"], 4), "gb_s": round(gguf_bytes / load["pinned"] / 1e9, 2),
                              "pageable_seconds": round(load["pageable"], 4),
                              "pageable_gb_s": round(gguf_bytes / load["pageable"] / 1e9, 2)}
    log(f"configs[3] load: {load['pinned']:.3f}s pinned staging, {load['pageable']:.3f}s pageable "
        f"({gguf_bytes / 1e9:.2f} GB)")
    gen = torch.Generator(device="cuda").manual_seed(7)
    for layer in range(cfg.layers):
        for value in (False, True):
            ptr, nbytes = s.kv_cache(layer, value)
            fill = torch.randn(nbytes // 2, generator=gen, device="cuda").half()
            assert hip.hipMemcpy(C.c_void_p(ptr), C.c_void_p(fill.data_ptr()), nbytes, 3) == 0
    torch.cuda.synchronize()
    s.set_position(4096)
    s.eval_greedy([11])
    s.decode(8, ids=False)             # warm-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    s.decode(128, ids=False)
    dt = time.perf_counter() - t0
    spec = synth.SPECS["qwen3-1.7b"]
    b = sum(spec.decode_bytes(4105 + i) for i in range(128))
    out["qwen3-1.7b_kv4096"] = {"workload": "configs[3]: Qwen3-1.7B-shape Q8_0, KV pre-filled to 4096, 128 greedy decode steps "
                                            "(order-exact spread attention)", "value": round(128 / dt, 2), "unit": "tok/s",
                                "hbm_frac": round(b / dt / HBM_PEAK, 4)}
    log(f"configs[3] decode at 4096: {128 / dt:.1f} tok/s")
    s.close()
    del s
    torch.cuda.empty_cache()
    f, cfg, table = model.load(synth.model_path("bitnet-2b"))
    p = synth.prompt_ids(64, cfg.vocab)
    s = HipSession((f, cfg, table), max_context=64 + 256 + 8)
    s.eval(p, logits=False)
    s.decode(8, ids=False)
    s.rollback(0)
    s.eval_greedy(p)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ids = s.decode(255)
    dt = time.perf_counter() - t0
    spec = synth.SPECS["bitnet-2b"]
    b = sum(spec.decode_bytes(64 + i) for i in range(255))
    entry = {"workload": "configs[4]: BitNet-b1.58-2B-shape TQ2_0 (x86 TQ2_0x16 arithmetic, 7-bit activations), "
                         "64-id prompt then 256 greedy tokens", "value": round(255 / dt, 2), "unit": "tok/s",
             "hbm_frac": round(b / dt / HBM_PEAK, 4)}
    golden = os.path.join(ROOT, "tests", "golden", "bitnet-2b_greedy.json")
    if os.path.exists(golden):
        with open(golden) as fh:
            want = json.load(fh)["ids"]
        n = min(len(want) - 1, len(ids))
        entry["greedy_matches_reference"] = bool(list(map(int, ids[:n])) == want[1:n + 1])
        entry["greedy_compared"] = n + 1
    out["bitnet-2b"] = entry
    log(f"configs[4] decode: {255 / dt:.1f} tok/s")
    s.close()
    return out


# The families that decode on the graph path (one kernel per phase, replayed from HIP graphs), at
# full-size shapes with synthetic weights (brisk_hip/synth.py names the dimensions).
FAMILY_SHAPES = (
    ("gemma3-1b", "Gemma-3-1B shape, Q4_0: sliding-window layers, post-norms, 256-wide heads (the plain attention)"),
    ("lfm2-1.2b", "LFM2-1.2B shape, Q4_0: 10 short-convolution layers, 6 attention layers"),
    ("qwen35-0.8b", "Qwen3.5 shape, Q4_0: 18 Gated DeltaNet layers (16 heads of 128x128 state), 6 gated attention "
                    "layers of 256-wide heads"),
    ("gemma4-e2b", "Gemma 4 shape, Q4_0: 35 layers, 256/512-wide heads, 15 shared K/V layers, 256-wide per-layer "
                   "embeddings (vocabulary cut to 65536)"),
)


def families(torch, HipSession, model, synth):
    """Decode tok/s of each graph-path family: a 32-id prompt, then 128 greedy steps; and a 512-id prompt.  hbm_frac counts the
    bytes of the weight matrices a token reads (each layer's, the output's, one embedding row) at HBM peak."""
    import numpy as np
    out = {}
    for name, desc in FAMILY_SHAPES:
        f, cfg, table = model.load(synth.model_path(name))
        tensors = {t.name: t for t in table}
        wbytes = sum(t.data.nbytes for t in table if t.rows > 1 and t.name not in ("token_embd.weight", "per_layer_token_embd.weight"))
        if "output.weight" not in tensors:  # tied: the embedding is the output projection
            wbytes += tensors["token_embd.weight"].data.nbytes
        p = synth.prompt_ids(32, cfg.vocab)
        s = HipSession((f, cfg, table), max_context=32 + 128 + 16)
        s.eval(p, logits=False)
        s.decode(8, ids=False)         # warm-up
        s.rollback(0)
        s.eval_greedy(p)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        s.decode(128, ids=False)
        dt = time.perf_counter() - t0
        out[name] = {"workload": desc + "; 32-id prompt, 128 greedy decode steps on the graph path",
                     "value": round(128 / dt, 2), "unit": "tok/s", "weight_bytes_per_token": int(wbytes),
                     "hbm_frac": round(wbytes * 128 / dt / HBM_PEAK, 4)}
        log(f"{name} decode: {128 / dt:.1f} tok/s")
        s.close()
        del s
        # a 512-id prompt (eval, last-token logits; median of 3), through the batched prefill
        lp = synth.prompt_ids(512, cfg.vocab, seed=11)
        s = HipSession((f, cfg, table), max_context=512 + 16)
        s.eval(lp[:64], logits=False)  # warm-up
        times = []
        for _ in range(3):
            s.rollback(0)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            s.eval(lp, logits=True)
            times.append(time.perf_counter() - t0)
        dtp = float(np.median(times))
        out[name]["prompt_512_tok_s"] = round(512 / dtp, 1)
        log(f"{name} 512-id prompt: {dtp * 1e3:.1f} ms -> {512 / dtp:.0f} tok/s")
        s.close()
        del s
        torch.cuda.empty_cache()
    return out


def profiled_traffic(steps):
    """HBM bytes of a `steps`-step decode launch measured by rocprofv3 (FETCH_SIZE + WRITE_SIZE, each scaled by a
    plain copy's reading), from the summary's `traffic_bytes_per_launch_K<steps>:` line (profiled for K = 256,
    the default, and K = 20, the driver's); None for a step count that was not profiled."""
    p = os.path.join(ROOT, "profiles", "k_loop_qwen3-0.6b_decode.md")
    if not os.path.exists(p):
        return None
    with open(p) as fh:
        for line in fh:
            if line.startswith(f"traffic_bytes_per_launch_K{steps}:"):
                return int(line.split(":")[1])
    return None


def copy_calibration(mb):
    import torch
    n = mb * (1 << 20) // 4
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n * 4}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-kernels", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip configs[3] (long context) and configs[4] (BitNet)")
    ap.add_argument("--no-families", action="store_true", help="skip the graph-path families' decode lines")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MB")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the token loop runs on a single device; a multi-GPU run would shard the layers' rows per GPU)", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return

    import numpy as np
    import torch
    from brisk_hip import HipSession, lib as L, model, synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    lib = L.load()
    name = "qwen3-0.6b"
    spec = synth.SPECS[name]
    t0 = time.time()
    path = synth.model_path(name)
    log(f"model {name}: {path} ({time.time() - t0:.1f}s)")
    f, cfg, table = model.load(path)
    prompt = synth.prompt_ids(32, cfg.vocab)
    K, W = args.steps, args.warmup
    t0 = time.time()
    s = HipSession((f, cfg, table), max_context=len(prompt) + max(K, W, 256) + 64)
    log(f"session load {time.time() - t0:.1f}s")

    # warmup: prompt + W steps, then back to the start of the workload
    s.eval(prompt, logits=False)
    s.decode(W, ids=False)
    s.rollback(0)
    first = s.eval_greedy(prompt)          # prompt evaluated (untimed), first pick pending
    st = torch.cuda.ExternalStream(s.stream)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(st)
    ids = s.decode(K)                      # K decode steps: one k_loop launch, one sync at the end
    ev1.record(st)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    loop_ms = ev0.elapsed_time(ev1)
    tok_s = K / dt
    ms_step = dt / K * 1e3
    gen = np.concatenate([[first], ids])
    step_bytes = [spec.decode_bytes(len(prompt) + i) for i in range(K)]
    launch_bytes = int(sum(step_bytes))
    mean_bytes = launch_bytes / K
    log(f"decode: {K} steps in {dt * 1e3:.1f} ms (k_loop {loop_ms:.1f} ms by events) -> {tok_s:.1f} tok/s, "
        f"{ms_step * 1e3:.1f} us/step, {mean_bytes / 1e6:.1f} MB/step -> {launch_bytes / (loop_ms * 1e-3) / 1e9:.1f} GB/s")
    # the whole configs[1] workload (256 steps after the prompt), whatever K is: its rate and its 256 ids
    FULL = 256
    if K == FULL:
        full_s, full_ids = dt, ids
    else:
        s.rollback(0)
        ffirst = s.eval_greedy(prompt)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        full_ids = s.decode(FULL)
        torch.cuda.synchronize()
        full_s = time.perf_counter() - t0
        gen_full = np.concatenate([[ffirst], full_ids])
    full_gen = gen if K == FULL else gen_full
    full_bytes = int(sum(spec.decode_bytes(len(prompt) + i) for i in range(FULL)))
    log(f"full workload: {FULL} steps in {full_s * 1e3:.1f} ms -> {FULL / full_s:.1f} tok/s")
    s.close()
    del s
    torch.cuda.empty_cache()

    result = {
        "metric": "decode tok/s (Qwen3-0.6B-shape Q4_0, greedy, on-device sampling)",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic (seeded random-weight GGUF)",
        "config": {"workload": "qwen3-0.6b-shape decode: 32 random prompt ids then greedy steps", "hidden": 1024,
                   "layers": 28, "heads": 16, "kv_heads": 8, "head_dim": 128, "ffn": 3072, "vocab": 151936,
                   "weights": "Q4_0 layers, Q8_0 embedding/output", "prompt": 32, "decode_steps": K},
        "roofline": {"kernel": "k_loop (persistent token loop; one launch = the K decode steps)", "bound": "hbm",
                     "achieved": round(launch_bytes / (loop_ms * 1e-3) / 1e9, 2), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(launch_bytes / (loop_ms * 1e-3) / HBM_PEAK, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": launch_bytes, "ms_per_launch": round(loop_ms, 3)},
    }
    traffic = profiled_traffic(K)
    if traffic is not None:
        result["roofline"]["traffic"] = traffic
        result["roofline"]["traffic_source"] = "profiles/k_loop_qwen3-0.6b_decode.md (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)"
    else:
        result["roofline"]["traffic_note"] = f"no rocprofv3 FETCH_SIZE/WRITE_SIZE pass on file for a {K}-step launch"
    result["full_workload"] = {"workload": "configs[1] as specified: 32-id prompt, then 256 greedy decode steps in one launch",
                               "value": round(FULL / full_s, 2), "unit": "tok/s", "ms_per_step": round(full_s / FULL * 1e3, 4),
                               "achieved_gb_s": round(full_bytes / full_s / 1e9, 2),
                               "frac": round(full_bytes / full_s / HBM_PEAK, 4)}
    golden = os.path.join(ROOT, "tests", "golden", "qwen3-0.6b_greedy.json")
    if os.path.exists(golden):
        with open(golden) as fh:
            want = json.load(fh)["ids"]
        n = min(len(full_gen), len(want))
        result["greedy_matches_reference"] = bool(list(map(int, full_gen[:n])) == want[:n])
        result["greedy_compared"] = n

    if not args.no_kernels:
        # 2048 x 2048 Q4_0, single launch (matrix cache-resident) and streamed over 128 copies
        ms0, algo0, g0 = gemv_roofline(torch, lib, L, 2048, 2048, 2, 18, copies=1, reps=512, norm=False, graph=True)
        ms1, algo1, g1 = gemv_roofline(torch, lib, L, 2048, 2048, 2, 18, copies=128, reps=512, norm=False, graph=True)
        ach1 = algo1 / (g1 * 1e-3) / 1e9
        # the same rows stacked 128 high in one matrix (302 MB): the kernel's streaming rate without per-launch latency
        ms2, algo2 = gemv_roofline(torch, lib, L, 128 * 2048, 2048, 2, 18, copies=1, reps=20, norm=False)
        ach2 = algo2 / (ms2 * 1e-3) / 1e9
        result["q4_0_gemv"] = {"config": "configs[0]: 2048x2048 Q4_0, x quantised to Q8_0 in-kernel",
                               "single_launch_us": round(g0 * 1e3, 2),
                               "streaming_us_per_launch": round(g1 * 1e3, 2), "streaming_copies": 128,
                               "timing": "launches replayed from a HIP graph (device time a launch); eager ctypes "
                                         "launches, bound by the host call: single %.2f us, streamed %.2f us" % (ms0 * 1e3, ms1 * 1e3),
                               "achieved": round(ach1, 1), "unit": "GB/s", "frac": round(ach1 / 8000.0, 4),
                               "algorithmic_bytes": algo1,
                               "one_launch_128_stacked": {"rows": 128 * 2048, "us": round(ms2 * 1e3, 2), "achieved": round(ach2, 1),
                                                          "frac": round(ach2 / 8000.0, 4), "algorithmic_bytes": algo2}}
        log(f"q4_0 gemv 2048x2048 (graph replay): single {g0 * 1e3:.2f} us, streamed {g1 * 1e3:.2f} us = {ach1:.0f} GB/s "
            f"(eager launches: {ms0 * 1e3:.2f} / {ms1 * 1e3:.2f} us); 128 copies stacked in one launch: "
            f"{ms2 * 1e3:.1f} us = {ach2:.0f} GB/s")
        ms, algo = gemv_roofline(torch, lib, L, cfg.vocab, cfg.embd, 8, 34, copies=2, reps=40, norm=True)
        ach = algo / (ms * 1e-3) / 1e9
        result["output_gemv"] = {"config": "151936x1024 Q8_0 with fused output_norm, 2 copies (330 MB)",
                                 "us_per_launch": round(ms * 1e3, 2), "achieved": round(ach, 1), "unit": "GB/s",
                                 "frac": round(ach / 8000.0, 4), "algorithmic_bytes": algo}
        log(f"output gemv: {ms * 1e3:.1f} us, {ach:.0f} GB/s")

    if not args.no_prefill:
        # Llama-3.2-1B-shape Q4_K_M, 512-id prefill (batched MFMA path), then 128 decode steps
        lname = "llama-3.2-1b"
        lpath = synth.model_path(lname)
        lf, lcfg, ltable = model.load(lpath)
        lp = synth.prompt_ids(512, lcfg.vocab, seed=11)
        ls = HipSession((lf, lcfg, ltable), max_context=1024)
        ls.eval(lp, logits=False)     # warm-up (untimed)
        times = []
        for _ in range(5):  # the median of five 512-token prompt evaluations
            ls.rollback(0)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            ls.eval(lp, logits=True)
            times.append(time.perf_counter() - t0)
        dtp = float(np.median(times))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ls.decode(128, ids=False)
        dtd = time.perf_counter() - t0
        # int8 ops of the layer contractions (q, k, v, o, gate, up, down), 2 per multiply-accumulate
        params = lcfg.layers * (2 * lcfg.embd * lcfg.heads * lcfg.head_dim + 2 * lcfg.embd * lcfg.kv_heads * lcfg.head_dim
                                + 3 * lcfg.embd * lcfg.ff)
        ops = 2 * 512 * params
        import ctypes as C
        tops, tops32 = C.c_double(), C.c_double()
        L.check(lib.brisk_hip_mfma_rate(0, C.byref(tops)))
        L.check(lib.brisk_hip_mfma_rate(1, C.byref(tops32)))
        log(f"int8 MFMA rate (register operands): v_mfma_i32_16x16x64_i8 {tops.value:.0f} TOP/s, "
            f"v_mfma_i32_32x32x32_i8 {tops32.value:.0f} TOP/s")
        result["prefill"] = {"workload": "configs[2]: llama-3.2-1b-shape Q4_K_M, 512 random prompt ids (eval, last-token logits; median of 5)",
                             "value": round(512 / dtp, 2), "unit": "tok/s", "ms": round(dtp * 1e3, 2),
                             "roofline": {"bound": "mfma", "achieved": round(ops / dtp / 1e12, 2), "peak": 5000.0,
                                          "unit": "TOP/s (int8)", "frac": round(ops / dtp / 5.0e15, 5),
                                          "ops": ops,
                                          "mfma_int8_measured_tops": round(tops.value, 1),
                                          "mfma_int8_32x32x32_measured_tops": round(tops32.value, 1),
                                          "frac_of_measured": round(ops / dtp / 1e12 / tops.value, 5)},
                             "decode_after_prefill_tok_s": round(128 / dtd, 2)}
        log(f"prefill 512: {dtp * 1e3:.1f} ms -> {512 / dtp:.1f} tok/s; then 128 decode steps {128 / dtd:.1f} tok/s")
        ls.rollback(0)
        base = ls.eval(lp, logits=True)
        ls.close()
        del ls
        # the same prompt with the opt-in MFMA attention (not order-exact)
        os.environ["BRISK_HIP_PREFILL_ATTN"] = "mfma"
        try:
            ms_ = HipSession((lf, lcfg, ltable), max_context=1024)
        finally:
            del os.environ["BRISK_HIP_PREFILL_ATTN"]
        ms_.eval(lp, logits=False)
        times = []
        for _ in range(5):
            ms_.rollback(0)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fast = ms_.eval(lp, logits=True)
            times.append(time.perf_counter() - t0)
        dtf = float(np.median(times))
        ms_.close()
        del ms_
        result["prefill"]["mfma_attention"] = {
            "note": "opt-in BRISK_HIP_PREFILL_ATTN=mfma: f16 MFMA attention (hi/lo operands), not order-exact",
            "value": round(512 / dtf, 2), "unit": "tok/s", "ms": round(dtf * 1e3, 2),
            "max_abs_logit_diff_vs_exact": float(np.abs(fast - base).max()),
            "argmax_equal": bool(int(np.argmax(fast)) == int(np.argmax(base)))}
        log(f"prefill 512 (mfma attention): {dtf * 1e3:.1f} ms -> {512 / dtf:.1f} tok/s, "
            f"max |diff| vs exact {np.abs(fast - base).max():.3g}")
        torch.cuda.empty_cache()

    if not args.no_configs:
        result["configs"] = other_configs(torch, HipSession, model, synth)
    if not args.no_families:
        result["families"] = families(torch, HipSession, model, synth)

    if not args.no_cpu_baseline:
        t0 = time.time()
        cb = cpu_baseline(path, prompt, 256)
        if cb is not None:
            ref_ids = cb.pop("ids")
            # the common prefix of the reference's 256 ids and the timed run's K + 1
            nc = min(len(ref_ids), len(full_gen))
            cb["greedy_matches_gpu"] = bool(np.array_equal(np.asarray(ref_ids[:nc]), full_gen[:nc]))
            cb["greedy_compared"] = int(nc)
            result["cpu_baseline"] = cb
            log(f"cpu baseline ({time.time() - t0:.1f}s): {cb['value']} tok/s on {cb['cores']} threads")
        else:
            result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
