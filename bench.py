"""Benchmark: the token sampler on BASELINE.json's configuration 5 (256 independent rows of 248,320
f32 logits, each with its own seed, 2,048-id history and parameters; the full penalty + top-k +
top-p + min-p chain) on one MI355X.

A step is one as_sample call over the 256-row batch, inputs already in HBM. Three copies of the
batch rotate between steps so no step finds its rows in the 256 MB Infinity Cache. The JSON line
also carries batch-1 latency (configs 2 and 3, one row per call), the scan kernel's roofline from
HIP events on the library's stream, and the CPU oracle timed on this host.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
CAL_FLOATS = 64 << 20  # the calibration copy: 256 MiB read, 256 MiB written
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "scan_kernel_config5_traffic.json")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def gpu_config5(steps, warmup, copies=3):
    import torch

    from artemis_amd import Context, PackedSampling, Sampling, states_tensor, workloads

    w = workloads.config5()
    dev = torch.device("cuda:0")
    params = [Sampling(p.temp, p.top_k, p.top_p, p.min_p, p.presence, p.frequency, p.repetition) for p in w.params]
    off, ids = w.hist_csr()
    rows, n = w.logits.shape
    host = torch.from_numpy(w.logits)
    sets = [host.to(dev) for _ in range(copies)]
    d_off = torch.from_numpy(off).to(dev)
    d_ids = torch.from_numpy(ids).to(dev)
    rng = states_tensor(w.seeds, dev)
    ctx = Context(max_rows=rows, max_vocab=n)
    # The settings array and the output buffers are made once, as the engine holds them: building a
    # 256-entry ctypes array from Python objects costs more than the kernels.
    packed = PackedSampling(params)
    out = ctx.outputs(rows)
    log(f"bench: config5 rows={rows} vocab={n} history={len(ids) // rows} digest={w.digest()}")
    # A plain elementwise kernel of known traffic (reads and writes 256 MiB), untimed: under
    # rocprofv3 --pmc its FETCH_SIZE / WRITE_SIZE calibrate the counters against known bytes.
    cal = torch.empty(CAL_FLOATS, dtype=torch.float32, device=dev).uniform_()
    torch.neg(cal, out=torch.empty_like(cal))
    torch.cuda.synchronize()
    del cal

    for i in range(warmup):
        ctx.sample_batch(sets[i % copies], packed, rng, d_off, d_ids, out=out)
    torch.cuda.synchronize()
    # The exact-order path rate on this batch (informational).
    tok, st, *_ = ctx.sample_batch(sets[0], packed, rng, d_off, d_ids, out=out)
    status = st.cpu().numpy()
    exact_rows = int(((status & 0x100) != 0).sum())

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        ctx.sample_batch(sets[i % copies], packed, rng, d_off, d_ids, out=out)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # The kernels' times in a second pass of the same steps: the profiling events sit between the
    # kernels and would slow the timed pass.
    ctx.profile(True)
    for i in range(steps):
        ctx.sample_batch(sets[i % copies], packed, rng, d_off, d_ids, out=out)
    scan_ms, finish_ms, calls = ctx.profile_read()
    ctx.profile(False)
    log(f"bench: {steps} steps in {wall * 1e3:.2f} ms; scan {scan_ms / calls * 1e3:.1f} us, "
        f"finish {finish_ms / calls * 1e3:.1f} us per call; exact-path rows {exact_rows}")
    hist_bytes = 4 * len(ids)
    alg_bytes = 4 * rows * n + hist_bytes
    ctx.close()
    return dict(rows=rows, n=n, wall=wall, scan_ms=scan_ms / calls, finish_ms=finish_ms / calls,
                alg_bytes=alg_bytes, exact_rows=exact_rows, digest=w.digest(), history=len(ids) // rows)


def gpu_batch1(reps=200):
    """One row per call, synchronised each time: µs per row at batch 1 (configs 2 and 3)."""
    import torch

    from artemis_amd import Context, PackedSampling, Sampling, states_tensor, workloads

    dev = torch.device("cuda:0")
    out = {}
    for name, w, s in [
        ("config2", workloads.config2(draws=1), Sampling(0.6, 20, 0.95, 0.0)),
        ("config3", workloads.config3(draws=1), Sampling(0.7, 40, 0.9, 0.05, 0.5, 0.3, 1.05)),
    ]:
        lg = torch.from_numpy(w.logits).to(dev)
        off, ids = w.hist_csr()
        d_off = torch.from_numpy(off).to(dev) if len(ids) else None
        d_ids = torch.from_numpy(ids).to(dev) if len(ids) else None
        ctx = Context(max_rows=1, max_vocab=lg.shape[1])
        rng = states_tensor([0], dev)
        packed, res = PackedSampling([s]), ctx.outputs(1)
        for _ in range(20):
            ctx.sample_batch(lg, packed, rng, d_off, d_ids, out=res)
        torch.cuda.synchronize()
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            tok, *_ = ctx.sample_batch(lg, packed, rng, d_off, d_ids, out=res)
            tok.item()
            times.append(time.perf_counter() - t0)
        ctx.profile(True)
        for _ in range(reps):
            ctx.sample_batch(lg, packed, rng, d_off, d_ids, out=res)
        scan_ms, finish_ms, calls = ctx.profile_read()
        ctx.close()
        t = np.array(times) * 1e6
        out[name] = dict(us_per_row_median=round(float(np.median(t)), 2), us_per_row_best=round(float(t.min()), 2),
                         kernel_us=round((scan_ms + finish_ms) / calls * 1e3, 2))
    return out


def gpu_logprobs(reps=50):
    """as_logprobs (logprobs.rs:12-38) at top 20: kernel time per call for config 5's 256 rows
    (HIP events on the library's stream, inputs rotated over three copies) and the wall time of one
    row per call."""
    import torch

    from artemis_amd import Context, workloads

    w = workloads.config5()
    dev = torch.device("cuda:0")
    rows, n = w.logits.shape
    host = torch.from_numpy(w.logits)
    sets = [host.to(dev) for _ in range(3)]
    tokens = torch.arange(rows, dtype=torch.int32, device=dev) * 7
    ctx = Context(max_rows=rows, max_vocab=n)
    for i in range(5):
        ctx.logprobs(sets[i % 3], tokens, 20)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        ctx.logprobs(sets[i % 3], tokens, 20)
    e1.record(stream)
    torch.cuda.synchronize()
    batch_us = e0.elapsed_time(e1) / reps * 1e3
    one = sets[0][:1]
    tok1 = tokens[:1]
    times = []
    for i in range(reps):
        t0 = time.perf_counter()
        lp, *_ = ctx.logprobs(one, tok1, 20)
        lp.cpu()
        times.append(time.perf_counter() - t0)
    ctx.close()
    alg = 4 * rows * n
    return dict(batch256_us=round(batch_us, 2), rows_per_s=round(rows / (batch_us * 1e-6), 1),
                hbm_frac=round(alg / (batch_us * 1e-6) / (HBM_PEAK_GBS * 1e9), 4),
                batch1_us_median=round(float(np.median(times)) * 1e6, 2))


def gpu_head(reps=30):
    """The output head (248,320 Q6_K rows of 2,048, decode.rs:850) as as_matvec (logits written) and
    as as_head_argmax (argmax_rows fused, no logits), then embed_rows of the draft: HIP events on the
    library's stream; weights 417 MB (past the 256 MB Infinity Cache, so every call reads HBM)."""
    import torch

    from artemis_amd import Context, WTYPE, row_bytes

    rows, k, q6 = 248_320, 2048, WTYPE["Q6_K"]
    rb = row_bytes(q6, k)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    w = torch.randint(0, 256, (rows, rb), dtype=torch.uint8, device=dev, generator=g)
    blocks = w.view(rows * (k // 256), 210)
    blocks[:, 208] = 0x00  # every block's f16 d = 2^-8: finite outputs
    blocks[:, 209] = 0x1C
    x = (torch.rand(k, device=dev, generator=g) * 2 - 1).contiguous()
    y = torch.empty(rows, dtype=torch.float32, device=dev)
    ids = torch.zeros(1, dtype=torch.int32, device=dev)
    addr = torch.zeros(1, dtype=torch.int64, device=dev)
    emb = w  # the embedding table: the head's own rows (tied), so every draft id has its row
    ctx = Context(max_rows=16, max_vocab=4096)
    stream = torch.cuda.current_stream()

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3

    mv_us = timed(lambda: ctx.matvec(w, q6, rows, k, x, y))
    ha_us = timed(lambda: ctx.head_argmax(w, q6, rows, k, x, ids, addr, emb.data_ptr(), rb))
    def draft_step():
        ctx.head_argmax(w, q6, rows, k, x, ids, addr, emb.data_ptr(), rb)
        ctx.embed_rows(addr, q6, k)

    chain_us = timed(draft_step)
    ctx.close()
    wbytes = rows * rb
    return dict(weights_bytes=wbytes,
                matvec_us=round(mv_us, 2), matvec_hbm_frac=round((wbytes + 4 * rows) / (mv_us * 1e-6) / (HBM_PEAK_GBS * 1e9), 4),
                head_argmax_us=round(ha_us, 2), head_argmax_hbm_frac=round(wbytes / (ha_us * 1e-6) / (HBM_PEAK_GBS * 1e9), 4),
                head_argmax_embed_us=round(chain_us, 2))


def cpu_baseline(budget_s=12.0):
    """The CPU oracle (the C++ restatement of the reference sampler) on this host: one row per call
    on one core, over a bounded sample of configuration 5's rows; and the 256 rows over all cores."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O

    from artemis_amd import workloads

    w = workloads.config5()
    params = [dict(temp=p.temp, top_k=p.top_k, top_p=p.top_p, min_p=p.min_p, presence=p.presence,
                   frequency=p.frequency, repetition=p.repetition) for p in w.params]
    off, ids = w.hist_csr()
    # One core: rows in order until the budget is spent (at least 32 rows).
    done, t0 = 0, time.perf_counter()
    chunk = 16
    while done < w.logits.shape[0] and (time.perf_counter() - t0 < budget_s / 2 or done < 32):
        sl = slice(done, done + chunk)
        sub_off = off[done:done + chunk + 1] - off[done]
        O.sample_rows(params[sl], w.seeds[sl], w.logits[sl], sub_off, ids[off[done]:off[min(done + chunk, len(params))]], threads=1)
        done += chunk
    one = time.perf_counter() - t0
    threads = min(os.cpu_count() or 1, 16)
    t1 = time.perf_counter()
    O.sample_rows(params, w.seeds, w.logits, off, ids, threads=threads)
    many = time.perf_counter() - t1
    return dict(one_core_rows_per_s=done / one, rows_sampled=done, all_cores_rows_per_s=w.logits.shape[0] / many,
                threads=threads)


def d2h_row_us(reps=50):
    """The reference copies each 993,280-byte row to the host before sampling (decode.rs:438)."""
    import torch

    from artemis_amd import workloads

    x = torch.empty(workloads.VOCAB, dtype=torch.float32, device="cuda")
    h = torch.empty(workloads.VOCAB, dtype=torch.float32, pin_memory=True)
    for _ in range(5):
        h.copy_(x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        h.copy_(x)
        torch.cuda.synchronize()
    return (time.perf_counter() - t0) / reps * 1e6


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU: the sampler's rows are independent and this build has no "
              f"multi-GPU path (asked for --gpus {a.gpus})", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)

    g = gpu_config5(a.steps, a.warmup)
    log("bench: batch-1 latency")
    b1 = gpu_batch1()
    log("bench: log-probabilities")
    lpb = gpu_logprobs()
    log("bench: output head")
    head = gpu_head()
    ms_per_step = g["wall"] / a.steps * 1e3
    rows_per_s = g["rows"] / (ms_per_step / 1e3)
    achieved = g["alg_bytes"] / (g["scan_ms"] / 1e3) / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        # HBM bytes per scan launch from the committed rocprofv3 --pmc passes over this same command.
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("scan_kernel_bytes_per_launch")
    cpu = None
    if not a.no_cpu:
        log("bench: CPU baseline")
        c = cpu_baseline()
        d2h = d2h_row_us()
        cpu = {"value": round(c["one_core_rows_per_s"], 2), "unit": "rows/s", "cores": 1, "kind": "port",
               "sample": f"the oracle (C++ restatement of sample.rs, -O2) on the first {c['rows_sampled']} "
                         f"config-5 rows, one fresh sampler and one draw per row, one core",
               "all_cores": {"value": round(c["all_cores_rows_per_s"], 2), "cores": c["threads"],
                             "sample": "all 256 config-5 rows, one row per task"},
               "d2h_copy_us_per_row": round(d2h, 2),
               "one_core_with_d2h_rows_per_s": round(1.0 / (1.0 / c["one_core_rows_per_s"] + d2h * 1e-6), 2)}
    out = {
        "metric": "sampled rows/s (248,320-vocab f32, 256-row batch, full penalty+top-k+top-p+min-p chain)",
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 logits, f64 probabilities",
        "data": "synthetic",
        "config": {"workload": "config5: 256 rows x 248,320 f32 logits, per-row seed, 2,048-id Zipf history, "
                               "T in [0.3,1], top-k in {0,20,50}, top-p in [0.8,1], min-p in [0,0.1], "
                               "rep 1.05 / presence 0.5 / frequency 0.3",
                   "rows": g["rows"], "vocab": g["n"], "history": g["history"], "input_digest": g["digest"],
                   "parallelism": "single GPU"},
        "us_per_row": round(ms_per_step * 1e3 / g["rows"], 4),
        "kernels_us": {"scan": round(g["scan_ms"] * 1e3, 2), "finish": round(g["finish_ms"] * 1e3, 2)},
        "exact_path_rows": g["exact_rows"],
        "batch1": b1,
        "logprobs_top20": lpb,
        "head_q6k_248320x2048": head,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "scan_kernel", "bytes_per_launch": g["alg_bytes"]},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
