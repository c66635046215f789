"""Benchmark: the token sampler on BASELINE.json's configuration 5 (256 independent rows of 248,320
f32 logits, each with its own seed, 2,048-id history and parameters; the full penalty + top-k +
top-p + min-p chain) on one MI355X.

A step is one as_sample call over the 256-row batch, inputs already in HBM. Three copies of the
batch rotate between steps so no step finds its rows in the 256 MB Infinity Cache. The JSON line
also carries batch-1 latency (configs 1-4: greedy, stochastic, penalised, and as_verify over 6 rows),
the roofline of the whole chain (every kernel of one as_sample call, HIP events on the library's
stream) with the scan kernel's share beside it, two worst-case 256-row batches (no filter at T = 1,
and min-p 0.002), and the CPU oracle timed on this host per
configuration, with and without the reference's device-to-host copy of each row.

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
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "sampler_chain_config5_traffic.json")


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
    # The rare paths' rates on this batch (informational).
    tok, st, *_ = ctx.sample_batch(sets[0], packed, rng, d_off, d_ids, out=out)
    status = st.cpu().numpy()
    exact_rows = int(((status & 0x100) != 0).sum())
    deep_rows = int(((status & 0x400) != 0).sum())

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
    scan_ms, rest_ms, calls = ctx.profile_read()
    ctx.profile(False)
    log(f"bench: {steps} steps in {wall * 1e3:.2f} ms; scan {scan_ms / calls * 1e3:.1f} us, "
        f"after the scan {rest_ms / calls * 1e3:.1f} us per call; exact-path rows {exact_rows}, deep {deep_rows}")
    hist_bytes = 4 * len(ids)
    alg_bytes = 4 * rows * n + hist_bytes
    ctx.close()
    return dict(rows=rows, n=n, wall=wall, scan_ms=scan_ms / calls, rest_ms=rest_ms / calls,
                alg_bytes=alg_bytes, exact_rows=exact_rows, deep_rows=deep_rows, digest=w.digest(),
                history=len(ids) // rows)


def gpu_batch1(reps=200):
    """One call per row (configs 1-3) or per verify step (config 4, 6 rows), synchronised each
    time: wall µs per call (median and best) and the kernels' µs per call (HIP events)."""
    import torch

    from artemis_amd import Context, PackedSampling, Sampling, states_tensor, workloads

    dev = torch.device("cuda:0")
    out = {}
    for name, w, s in [
        ("config1", workloads.config1(), Sampling(0.0, 0, 1.0, 0.0)),
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
        scan_ms, rest_ms, calls = ctx.profile_read()
        ctx.close()
        t = np.array(times) * 1e6
        out[name] = dict(us_per_row_median=round(float(np.median(t)), 2), us_per_row_best=round(float(t.min()), 2),
                         kernel_us=round((scan_ms + rest_ms) / calls * 1e3, 2))
    # Config 4: as_verify over k + 1 = 6 rows (5 drafts), T 0.6, top-p 0.95, the same stream state
    # each call.
    w = workloads.config4()
    rows = torch.from_numpy(w.logits).to(dev)
    drafts = torch.from_numpy(w.drafts.astype(np.int32)).to(dev)
    ctx = Context(max_rows=8, max_vocab=rows.shape[1])
    s = Sampling(0.6, 0, 0.95, 0.0)
    st0 = states_tensor([1234], dev)
    rng = st0.clone()
    for _ in range(10):
        rng.copy_(st0)
        ctx.verify(rows, drafts, s, rng)
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        rng.copy_(st0)
        t0 = time.perf_counter()
        _, result = ctx.verify(rows, drafts, s, rng)
        res = result.cpu()
        times.append(time.perf_counter() - t0)
    ctx.profile(True)
    for _ in range(reps):
        rng.copy_(st0)
        ctx.verify(rows, drafts, s, rng)
    scan_ms, rest_ms, calls = ctx.profile_read()
    ctx.close()
    t = np.array(times) * 1e6
    out["config4"] = dict(rows=int(rows.shape[0]), read=int(res[0]), accepted=int(res[1]),
                          us_per_call_median=round(float(np.median(t)), 2), us_per_call_best=round(float(t.min()), 2),
                          kernel_us=round((scan_ms + rest_ms) / calls * 1e3, 2))
    return out


def gpu_worst(reps=10):
    """Batches that config 5 does not reach: 256 rows of config 5's logits (no history) with no
    filter at T = 1 (every draw's total is the whole row's, and a draw may land past the sorted
    candidates), and 256 rows with min-p 0.002 and no top-k (floor sets of thousands of values).
    Per call: the chain's kernel time (HIP events on the library's stream) and how many rows took
    the rare paths."""
    import torch

    from artemis_amd import Context, PackedSampling, Sampling, states_tensor, workloads

    w = workloads.config5()
    dev = torch.device("cuda:0")
    rows, n = w.logits.shape
    host = torch.from_numpy(w.logits)
    sets = [host.to(dev) for _ in range(3)]
    ctx = Context(max_rows=rows, max_vocab=n)
    out = {}
    for name, s in [("unfiltered_t1", Sampling(1.0, 0, 1.0, 0.0)), ("minp_0.002", Sampling(0.7, 0, 1.0, 0.002))]:
        packed, res = PackedSampling([s] * rows), ctx.outputs(rows)
        rng = states_tensor(w.seeds, dev)
        for i in range(2):
            ctx.sample_batch(sets[i % 3], packed, rng, out=res)
        _, st, *_ = ctx.sample_batch(sets[0], packed, rng, out=res)
        status = st.cpu().numpy()
        ctx.profile(True)
        for i in range(reps):
            ctx.sample_batch(sets[i % 3], packed, rng, out=res)
        scan_ms, rest_ms, calls = ctx.profile_read()
        ctx.profile(False)
        out[name] = dict(us_per_call=round((scan_ms + rest_ms) / calls * 1e3, 2),
                         scan_us=round(scan_ms / calls * 1e3, 2), after_scan_us=round(rest_ms / calls * 1e3, 2),
                         deep_rows=int(((status & 0x400) != 0).sum()), exact_rows=int(((status & 0x100) != 0).sum()),
                         tail_pass_rows=int(((status & 0x800) != 0).sum()))
    ctx.close()
    return out


def gpu_cliffs(reps=5):
    """The paths config 5 does not take, timed. Top-k past the one-pass limit (k = 1,000, 10,000 and
    248,319; sample.rs:296-299 gives the reference's CPU times for these), at T = 1 with no other
    filter and no penalties, for one row (config 5's row 0) and for config 5's 256 rows; beside each,
    the CPU oracle's µs for one row at the same k, one core. And config 5's workload drawn with
    16,000-id histories (more distinct ids per slice than the scan's hash holds). Kernel µs per call (HIP events on the
    library's stream) and the rows that took the exact path."""
    import torch

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O

    from artemis_amd import Context, PackedSampling, Sampling, states_tensor, workloads

    w = workloads.config5()
    dev = torch.device("cuda:0")
    rows, n = w.logits.shape
    host = torch.from_numpy(w.logits)
    lg = host.to(dev)

    def timed(ctx, logits, packed, rng, res, off=None, ids=None):
        for _ in range(2):
            ctx.sample_batch(logits, packed, rng, off, ids, out=res)
        _, st, *_ = ctx.sample_batch(logits, packed, rng, off, ids, out=res)
        status = st.cpu().numpy()
        ctx.profile(True)
        for _ in range(reps):
            ctx.sample_batch(logits, packed, rng, off, ids, out=res)
        scan_ms, rest_ms, calls = ctx.profile_read()
        ctx.profile(False)
        return dict(us_per_call=round((scan_ms + rest_ms) / calls * 1e3, 2), scan_us=round(scan_ms / calls * 1e3, 2),
                    exact_rows=int(((status & 0x100) != 0).sum()), deep_rows=int(((status & 0x400) != 0).sum()))

    out = {}
    ctx1, ctx = Context(max_rows=1, max_vocab=n), Context(max_rows=rows, max_vocab=n)
    row0 = np.ascontiguousarray(w.logits[0])
    for k in (1000, 10000, 248319):
        s = Sampling(1.0, k, 1.0, 0.0)
        one = timed(ctx1, lg[:1], PackedSampling([s]), states_tensor([w.seeds[0]], dev), ctx1.outputs(1))
        batch = timed(ctx, lg, PackedSampling([s] * rows), states_tensor(w.seeds, dev), ctx.outputs(rows))
        cpu = []
        for i in range(3 if k > 10000 else 10):
            smp = O.Sampler(w.seeds[0], temp=1.0, top_k=k, top_p=1.0, min_p=0.0)
            cpu.append(smp.sample_timed(row0)[1] / 1e3)
        out[f"topk_{k}"] = dict(batch1=one, batch256=batch, cpu_oracle_us_one_row=round(float(np.median(cpu)), 1))
    ctx1.close()
    wh = workloads.config5(hist=16000)
    off, ids = wh.hist_csr()
    params = PackedSampling([Sampling(p.temp, p.top_k, p.top_p, p.min_p, p.presence, p.frequency, p.repetition)
                             for p in wh.params])
    lgh = torch.from_numpy(wh.logits).to(dev)
    out["history_16000"] = timed(ctx, lgh, params, states_tensor(wh.seeds, dev), ctx.outputs(rows),
                                 torch.from_numpy(off).to(dev), torch.from_numpy(ids).to(dev))
    ctx.close()
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


def cpu_baseline(reps=100):
    """The CPU oracle (the C++ restatement of the reference sampler, -O3) on this host, per
    configuration, one row (config 4: one verify step) per call on one core: the engine's per-row
    work (the non-finite check and Sampler::sample; config 4 the verify loop) timed in C, median and
    best of `reps` calls after a warm-up, alone and with the device-to-host copy of each row read
    that the reference pays first (decode.rs:438, verify.rs:345), timed here from a GPU buffer into
    pinned host memory. Config 5 cycles through its 256 rows. Also config 5's 256 rows over all
    cores, one row per task."""
    import torch

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O

    from artemis_amd import workloads

    def settings(p):
        return dict(temp=p.temp, top_k=p.top_k, top_p=p.top_p, min_p=p.min_p, presence=p.presence,
                    frequency=p.frequency, repetition=p.repetition)

    def stats(ns, copy_us):
        c = np.array(ns) / 1e3
        t = c + np.array(copy_us)
        return dict(median_us=round(float(np.median(c)), 2), best_us=round(float(c.min()), 2),
                    mean_us=round(float(c.mean()), 2),
                    median_with_d2h_us=round(float(np.median(t)), 2), best_with_d2h_us=round(float(t.min()), 2))

    dev = torch.device("cuda:0")
    per = {}
    for name, w in [("config1", workloads.config1()), ("config2", workloads.config2(draws=reps + 5)),
                    ("config3", workloads.config3(draws=reps + 5)), ("config5", workloads.config5())]:
        gpu_rows = torch.from_numpy(w.logits).to(dev)
        host = torch.empty(w.logits.shape[1], dtype=torch.float32, pin_memory=True)
        hview = host.numpy()
        ns, copy = [], []
        for i in range(reps + 5):
            r = i % len(w.params)
            smp = O.Sampler(w.seeds[r], **settings(w.params[r]))
            if w.histories and len(w.histories[r]):
                smp.add_history(w.histories[r])
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            host.copy_(gpu_rows[i % w.logits.shape[0]])
            torch.cuda.synchronize()
            cu = (time.perf_counter() - t0) * 1e6
            _, t = smp.sample_timed(hview)
            if i >= 5:
                ns.append(t)
                copy.append(cu)
        per[name] = stats(ns, copy)
        del gpu_rows
    # Config 4: the verify loop over 6 rows (it stops at the first pick that differs from its draft).
    w = workloads.config4()
    gpu_rows = torch.from_numpy(w.logits).to(dev)
    host = torch.empty(w.logits.shape, dtype=torch.float32, pin_memory=True)
    ns, copy = [], []
    picks = []
    for i in range(reps + 2):
        smp = O.Sampler(w.seeds[0], temp=0.6, top_k=0, top_p=0.95, min_p=0.0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        host.copy_(gpu_rows)
        torch.cuda.synchronize()
        cu = (time.perf_counter() - t0) * 1e6
        picks, t = smp.verify_timed(host.numpy(), list(w.drafts))
        if i >= 2:
            ns.append(t)
            copy.append(cu)
    per["config4"] = stats(ns, copy)
    per["config4"]["rows_read"] = len(picks)
    # Config 5's batch over all cores.
    w = workloads.config5()
    off, ids = w.hist_csr()
    params = [settings(p) for p in w.params]
    # The box gives one GPU's job a 16-core share of its host (whatever os.cpu_count() shows).
    threads = min(len(os.sched_getaffinity(0)), 16)
    t1 = time.perf_counter()
    O.sample_rows(params, w.seeds, w.logits, off, ids, threads=threads)
    many = time.perf_counter() - t1
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    host = dict(cpu_model=model, os_cpu_count=os.cpu_count(), affinity=len(os.sched_getaffinity(0)),
                omp_num_threads=os.environ.get("OMP_NUM_THREADS"))
    return dict(per_config=per, all_cores_rows_per_s=w.logits.shape[0] / many, threads=threads, host=host)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only-config5", action="store_true", help="only the config-5 steps (for profiling)")
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
    b1 = lpb = head = worst = cliffs = None
    if not a.only_config5:
        log("bench: batch-1 latency")
        b1 = gpu_batch1()
        log("bench: worst-case batches")
        worst = gpu_worst()
        log("bench: top-k past 256 and long histories")
        cliffs = gpu_cliffs()
        log("bench: log-probabilities")
        lpb = gpu_logprobs()
        log("bench: output head")
        head = gpu_head()
    ms_per_step = g["wall"] / a.steps * 1e3
    rows_per_s = g["rows"] / (ms_per_step / 1e3)
    chain_ms = g["scan_ms"] + g["rest_ms"]
    achieved = g["alg_bytes"] / (chain_ms / 1e3) / 1e9
    scan_achieved = g["alg_bytes"] / (g["scan_ms"] / 1e3) / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        # HBM bytes per call of the chain from the committed rocprofv3 --pmc passes over this command.
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("chain_bytes_per_call")
    cpu = None
    if not a.no_cpu and not a.only_config5:
        log("bench: CPU baseline")
        c = cpu_baseline()
        c5 = c["per_config"]["config5"]
        cpu = {"value": round(1e6 / c5["mean_us"], 2), "unit": "rows/s", "cores": 1, "kind": "port",
               "sample": "the oracle (C++ restatement of sample.rs, -O3): 100 config-5 rows in turn, one fresh "
                         "sampler with the row's history and one draw each, the non-finite check and the "
                         "sample timed, one core",
               "per_config_us": c["per_config"],
               "all_cores": {"value": round(c["all_cores_rows_per_s"], 2), "cores": c["threads"],
                             "sample": "all 256 config-5 rows, one row per task, on the job's share of "
                                       "the host (16 cores for one GPU)"},
               "host": c["host"]}
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
        "kernels_us": {"chain": round(chain_ms * 1e3, 2), "scan": round(g["scan_ms"] * 1e3, 2),
                       "after_scan": round(g["rest_ms"] * 1e3, 2)},
        "exact_path_rows": g["exact_rows"],
        "deep_path_rows": g["deep_rows"],
        "batch1": b1,
        "worst_case_batches": worst,
        "cliffs": cliffs,
        "logprobs_top20": lpb,
        "head_q6k_248320x2048": head,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "the as_sample chain: every kernel of one call (scan, finish)",
                     "bytes_per_launch": g["alg_bytes"],
                     "scan_only": {"achieved": round(scan_achieved, 1), "frac": round(scan_achieved / HBM_PEAK_GBS, 4)}},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
