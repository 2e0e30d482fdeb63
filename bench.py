"""GPT-2 124M fwd+bwd+AdamW training step on one MI355X ('hip' device).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload: GPT-2 small, fp32, 12 layers, 12 heads, d=768, vocab 50257,
context 1024, tied embeddings, random-init weights N(0, 0.02) (biases 0,
LayerNorm 1/0); batch 8 x 1024 synthetic tokens uniform in [0, 50257);
next-token cross_entropy; full backward; AdamW(lr 6e-4, wd 0.1).

Prints ONE JSON line.  `value` = tokens/s over exactly K timed steps
(inputs resident in HBM, device synchronised on both sides of the timed
region).  `roofline` reports the dominant kernel family (the MFMA GEMMs of
the Linear layers) from the start / stop timestamps of each of its
kernels' own dispatches (hipExtLaunchKernel events: no marker packets
between launches) over K more steps right after the timed region, the
same work (the timestamps cost ~10 us of issue time per launch, so they
stay out of the region that gives `value`); `roofline.traffic` is the HBM bytes
per launch measured by rocprofv3 counters
(profiles/gemm_hbm_traffic_gpt2.json).  `hbm_kernels` and
`kernel_ms_per_step` come from a pass after the timed region in which
every kernel carries such timestamps (the sums are kernel execution time,
as a kernel trace reports it).  `public_api` times the same model written
with the public operators only (nn.Linear, F.gelu, `+`), which do not
reach the fused GEMM epilogues.  `workloads` holds the four other
configurations' lines (MLP, elementwise chain, CNN, transformer block).
`cpu_baseline` times the oracle (numpy) on a bounded sample of the same
workload on the host.

    python bench.py --config mlp|chain|cnn|block   # the other four workloads
    python bench.py --copy-mib 1024      # known-size copy for counter scaling
    python bench.py --summarize-pmc FETCH WRITE COPY_FETCH COPY_WRITE
        # rocprofv3 --pmc output dirs -> profiles/gemm_hbm_traffic_gpt2.json
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GPT-2 124M fwd+bwd+AdamW tokens/s (1 GPU); bwd-kernel HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
DOMINANT = "gemm"  # kernel family of the Linear-layer GEMMs (k_gemm + split-K reduce)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_hbm_traffic_gpt2.json")
FP32_MFMA_PEAK_TFLOPS = 157.3

V, CTX, D, H, LAYERS = 50257, 1024, 768, 12, 12
B, T = 8, 1024


def linear_flops_per_step(b, t):
    """Algorithmic FLOPs of the Linear-layer GEMMs in one fwd+bwd step:
    2*tokens*in*out per product, three products (y, dx, dW) per layer."""
    tok = b * t
    per_layer = D * 3 * D + D * D + D * 4 * D + 4 * D * D
    fwd = 2 * tok * (LAYERS * per_layer + D * V)
    return 3 * fwd


def hbm_bytes_per_step(b, t, nparams, distinct_ids):
    """Algorithmic HBM bytes (inputs read once + outputs written once) per
    step for the memory-bound backward kernel families."""
    tok = b * t
    f = 4
    return {
        # the loss and dlogits = (softmax - onehot) / rows in one pass
        # (loss.backward()'s unit seed): read logits, write dlogits
        "cross_entropy_fwd_grad": 2 * tok * V * f,
        # the same gradient for another upstream gradient, after the forward
        "cross_entropy_bwd": 2 * tok * V * f,
        # 25 LayerNorms: read dy, x; write dx (+ mean/rstd, gamma); the 24
        # in the blocks also read the residual stream's gradient, which they
        # add into dx (GELU's backward runs in a GEMM epilogue: no kernel)
        "layer_norm_bwd": (2 * LAYERS + 1) * (3 * tok * D * f + 2 * tok * f + D * f) +
                          2 * LAYERS * tok * D * f,
        # AdamW: read p, g, m, v; write p, m, v
        "adam": 7 * nparams * f,
        # embedding backward, both tables in one launch: dout read once, the
        # token table's distinct rows of the tied head gradient read and
        # written, the ids read, the position table's T rows written
        "embedding_bwd": tok * D * f + 2 * distinct_ids * D * f + tok * 4 + t * D * f,
    }


def run_gpu(steps, warmup):
    import __graft_entry__ as ge
    torch = ge.load_package()
    from torchjs_amd import workloads as W
    torch.init(0)
    torch.manual_seed(1234)
    model = W.GPT2(V, CTX, D, H, LAYERS)
    print("gpt2: model built", file=sys.stderr, flush=True)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith(("ln_1.weight", "ln_2.weight")) or name == "ln_f.weight":
                p.fill_(1.0)
            elif name.endswith("bias"):
                p.zero_()
            else:
                p.copy_(torch.randn(*p.shape) * 0.02)
    nparams = sum(p.numel() for p in model.parameters())
    opt = torch.optim.AdamW(model.parameters(), lr=6e-4, weight_decay=0.1)
    rng = np.random.default_rng(1234)
    toks = rng.integers(0, V, (B, T + 1)).astype(np.int32)
    ids = torch.tensor(toks[:, :-1])
    tgt = torch.tensor(toks[:, 1:])

    rf = torch.profiler.record_function

    def step():
        # the phases are roctx ranges (rocprofv3 --marker-trace shows them)
        opt.zero_grad()
        with rf("gpt2.forward"):
            loss = model.loss(ids, tgt)
        with rf("gpt2.backward"):
            loss.backward()
        with rf("gpt2.adamw"):
            opt.step()
        return loss

    for i in range(warmup):
        loss = step()
        print("warmup %d loss %.4f" % (i, loss.item()), file=sys.stderr, flush=True)
    torch.synchronize()
    # timed region: K steps with no instrumentation (a timestamped dispatch
    # costs ~10 us of issue time, 2.5% of a step when every GEMM carries one)
    torch.hip.kernel_timing(False)
    torch.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    torch.synchronize()
    elapsed = time.perf_counter() - t0
    final_loss = loss.item()
    # roofline pass: the same K steps again, the dominant family's kernels
    # carrying their dispatch start / stop timestamps
    torch.hip.kernel_timing(True, only=DOMINANT)
    torch.hip.kernel_timing_reset()
    for _ in range(steps):
        step()
    dominant = torch.hip.kernel_time(DOMINANT)
    # pass after the timed region with every kernel timestamped, for the
    # per-family breakdown
    prof_steps = max(1, min(steps, 5))
    torch.hip.kernel_timing(True)
    torch.hip.kernel_timing_reset()
    for _ in range(prof_steps):
        step()
    fams = torch.hip.kernel_families()
    timing = {f: torch.hip.kernel_time(f) for f in fams}
    torch.hip.kernel_timing(False)
    mem = torch.hip.memory_stats()
    public = public_api_rate(torch, W, model, ids, tgt, min(steps, 5))
    distinct = int(np.unique(toks[:, :-1]).size)
    return elapsed, final_loss, dominant, timing, prof_steps, nparams, mem, public, distinct


def public_api_rate(torch, W, fused_model, ids, tgt, steps):
    """The same GPT-2 step with the model written in the public operators
    only (nn.Linear, F.gelu, `+`): the GELU and residual adds run as their
    own kernels instead of in the GEMM epilogues."""
    model = W.GPT2(V, CTX, D, H, LAYERS, fused=False)
    model.load_state_dict(fused_model.state_dict())
    opt = torch.optim.AdamW(model.parameters(), lr=6e-4, weight_decay=0.1)

    def step():
        opt.zero_grad()
        loss = model.loss(ids, tgt)
        loss.backward()
        opt.step()
        return loss
    for _ in range(2):
        step()
    torch.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.synchronize()
    el = time.perf_counter() - t0
    print("gpt2 public API: %.1f tokens/s" % (B * T * steps / el), file=sys.stderr, flush=True)
    return {"value": round(B * T * steps / el, 1), "unit": "tokens/s", "steps": steps,
            "ms_per_step": round(1000.0 * el / steps, 3),
            "model": "GPT-2 124M from nn.Linear, F.gelu and `+` (no epilogue fusion)"}


def _host():
    """Host CPU facts for the CPU baseline."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        threads = 1
    return {"host_cores": os.cpu_count() or 1, "host_cores_available": avail, "cpu_model": model,
            "threads_used": int(threads)}


def cpu_baseline():
    """The oracle (numpy) on a bounded sample: GPT-2 small at B=1, T=1024,
    full 12 layers and vocabulary, fwd + bwd + AdamW."""
    from oracle import models as om
    host = _host()
    cfg = om.Config()
    r = np.random.default_rng(0)
    p = om.init_params(cfg, r)
    tb, tt = 1, 1024
    ids = r.integers(0, V, (tb, tt + 1))
    t0 = time.perf_counter()
    _, g = om.gpt2_loss_and_grads(cfg, p, ids[:, :-1], ids[:, 1:])
    om.adamw_step(p, g, lr=6e-4, wd=0.1, step=1)
    dt = time.perf_counter() - t0
    out = {"value": round(tb * tt / dt, 2), "unit": "tokens/s", "cores": host["threads_used"],
           "kind": "port",
           "sample": "oracle (numpy float64, multithreaded BLAS) GPT-2 124M fwd+bwd+AdamW at "
                     "B=1, T=1024 (1024 tokens, full 12 layers and 50257 vocab), %.1f s" % dt}
    out.update(host)
    return out


def traffic_per_launch():
    """HBM bytes per launch of the dominant family, from the rocprofv3
    FETCH_SIZE / WRITE_SIZE summary kept under profiles/ (each counter
    scaled by what it reads for a plain copy of known size), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return int(t["hbm_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def copy_calibration(mib):
    """A plain contiguous device copy of `mib` MiB through the library's
    vectorised copy kernel (3 launches): the known-size reference that HBM
    byte counters are scaled by."""
    import __graft_entry__ as ge
    torch = ge.load_package()
    torch.init(0)
    n = mib * (1 << 20) // 4
    x = torch.zeros(n)
    for _ in range(3):
        y = x.clone()
    torch.synchronize()
    del y
    print(json.dumps({"copy_calibration_bytes": n * 4, "launches": 3}), flush=True)


# ------------------------------------------------------------ other workloads

CONFIGS = {
    "mlp": "MLP 784-256-ReLU-10 train step, batch 64, cross_entropy, Adam(lr 1e-3)",
    "chain": "x[4096,4096] + bias[4096] -> GELU -> * y -> sum(0) -> mean, fwd+bwd",
    "cnn": "CNN [32,3,64,64]: conv 3->32 3x3 p1, ReLU, conv 32->64 3x3 s2 p1, ReLU, "
           "avg-pool, Linear(64,10), cross_entropy, fwd+bwd",
    "block": "pre-LN transformer block B=8 T=1024 d=768 12 heads causal, 4x GELU MLP, "
             "loss=mean, fwd+bwd",
}

# timed steps of each workload inside the default run (each well under a second)
WORKLOAD_STEPS = {"mlp": 50, "chain": 20, "cnn": 20, "block": 10}

# algorithmic work per step (the roofline numerators)
MLP_FLOPS = 2 * 64 * (784 * 256 + 256 * 10) + 2 * 64 * (784 * 256 + 2 * 256 * 10)
MLP_ADAM_BYTES = 28 * (784 * 256 + 256 + 256 * 10 + 10)
CHAIN_FUSED_BYTES = 4 * 4096 * 4096 * 4 + 2 * 4096 * 4  # read x, y; write gx, gy; bias, gbias
CNN_FLOPS = 226492416 + 3 * 1207959552 + 226492416 + 3 * 40960
BLOCK_FLOPS = 3 * (2 * 8192 * (768 * 2304 + 768 * 768 + 2 * 768 * 3072) +
                   4 * 8 * 12 * 64 * (1024 * 1025 // 2))


def _replayed(torch, step, steps):
    """Seconds per step of `step` captured in a HIP graph and replayed (all
    of its kernels, one launch per replay), or None when it cannot be
    captured."""
    g = torch.hip.Graph()
    try:
        with torch.hip.graph(g):
            step()
    except Exception as e:  # a step that reads back to the host stays eager
        print("graph capture failed: %s" % e, file=sys.stderr, flush=True)
        return None
    for _ in range(3):
        g.replay()
    torch.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.synchronize()
    el = time.perf_counter() - t0
    g.reset()
    return el / steps


def _timed(torch, step, steps, warmup, graph=False):
    """(seconds per step, per-family kernel ms).  With `graph`, the step is
    also captured and replayed; returns (graph s, per, eager s)."""
    for _ in range(warmup):
        step()
    torch.synchronize()
    torch.hip.kernel_timing(False)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.synchronize()
    el = time.perf_counter() - t0
    replay = _replayed(torch, step, steps) if graph else None
    # instrumented pass after the timed region: per-family kernel time
    torch.hip.kernel_timing(True)
    torch.hip.kernel_timing_reset()
    for _ in range(steps):
        step()
    fams = {f: torch.hip.kernel_time(f) for f in torch.hip.kernel_families()}
    torch.hip.kernel_timing(False)
    per = {f: round(ms / steps, 4) for f, (n, ms) in sorted(fams.items(), key=lambda x: -x[1][1])
           if ms > 0}
    if graph:
        return (replay if replay is not None else el / steps), per, el / steps
    return el / steps, per


def _cpu_time(fn):
    t0 = time.perf_counter()
    fn()
    return time.perf_counter() - t0


def run_config(name, steps, warmup, cpu):
    import __graft_entry__ as ge
    torch = ge.load_package()
    from torchjs_amd import workloads as W
    from oracle import models as om
    from oracle import ops
    from oracle.rng import Generator
    torch.init(0)
    out = {"metric": name, "config": {"workload": CONFIGS[name]}, "n_gpus": 1, "steps": steps,
           "warmup": warmup, "dtype": "f32", "data": "synthetic (seeded host generator)"}
    if name == "mlp":
        g = Generator(1234)
        x = g.randn((64, 784))
        t = g.integers((64,), 10)
        model = W.mlp()
        # device step counters: the same update bit for bit, and capturable
        opt = torch.optim.Adam(model.parameters(), lr=1e-3, capturable=True)
        tx, tt = torch.tensor(x), torch.tensor(t)

        def step():
            opt.zero_grad()
            torch.F.cross_entropy(model(tx), tt).backward()
            opt.step()
        sec, per, eager = _timed(torch, step, steps, warmup, graph=True)
        out.update({"metric": "MLP train step samples/s", "value": round(64 / sec, 1),
                    "unit": "samples/s", "us_per_step": round(sec * 1e6, 1),
                    "timing": ("HIP graph replay of the whole step (hip.Graph)" if sec != eager
                               else "eager (the step could not be captured)"),
                    "eager": {"value": round(64 / eager, 1), "us_per_step": round(eager * 1e6, 1)},
                    "roofline": {"bound": "launch", "gemm_TFLOP/s": round(MLP_FLOPS / sec / 1e12, 4),
                                 "adam_GB/s": round(MLP_ADAM_BYTES / sec / 1e9, 2)}})
        if cpu:
            p = {k: v.numpy() for k, v in model.named_parameters()}

            def ref():
                _, gr = om.mlp_loss_and_grads(p, x, t)
                for k in p:
                    ops.adam_step(p[k], gr[k], np.zeros_like(p[k]), np.zeros_like(p[k]), 1, lr=1e-3)
            dt = _cpu_time(ref)
            out["cpu_baseline"] = {"value": round(64 / dt, 1), "unit": "samples/s", "kind": "port",
                                   "sample": "oracle (numpy float64), full config, one step"}
    elif name == "chain":
        g = Generator(99)
        n = 4096
        x, b, y = g.randn((n, n)), g.randn((n,)), g.uniform((n, n), -1, 1)
        tx, tb, ty = (torch.tensor(a, requires_grad=True) for a in (x, b, y))

        def step():
            for t_ in (tx, tb, ty):
                t_.grad = None
            W.chain_loss(tx, tb, ty).backward()
        sec, per, eager = _timed(torch, step, steps, warmup, graph=True)
        out.update({"metric": "elementwise+reduction fwd+bwd GB/s (fused-minimum bytes)",
                    "value": round(CHAIN_FUSED_BYTES / sec / 1e9, 1), "unit": "GB/s",
                    "ms_per_step": round(sec * 1e3, 3),
                    "timing": ("HIP graph replay of the whole step (hip.Graph)" if sec != eager
                               else "eager (the step could not be captured)"),
                    "eager": {"value": round(CHAIN_FUSED_BYTES / eager / 1e9, 1),
                              "ms_per_step": round(eager * 1e3, 3)},
                    "roofline": {"bound": "hbm", "achieved": round(CHAIN_FUSED_BYTES / sec / 1e9, 1),
                                 "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                 "frac": round(CHAIN_FUSED_BYTES / sec / 1e9 / HBM_PEAK_GBS, 3),
                                 "note": "end to end over the fused minimum (read x, y; write "
                                         "gx, gy): one pass (expr_colsum3) forms the loss's "
                                         "column sum, x's and y's gradients and the bias "
                                         "gradient; then the loss's mean and the small "
                                         "launches of the step"},
                    "kernels": {f: {"ms_per_step": ms, "GB/s": round(CHAIN_FUSED_BYTES / ms / 1e6, 1),
                                    "frac": round(CHAIN_FUSED_BYTES / ms / 1e6 / HBM_PEAK_GBS, 3)}
                                for f, ms in per.items() if f.startswith("expr")}})
        if cpu:
            dt = _cpu_time(lambda: om.chain_loss_and_grads(x, b, y))
            out["cpu_baseline"] = {"value": round(CHAIN_FUSED_BYTES / dt / 1e9, 2), "unit": "GB/s",
                                   "kind": "port", "sample": "oracle (numpy float64), full 4096^2"}
    elif name == "cnn":
        g = Generator(7)
        x = g.randn((32, 3, 64, 64))
        t = g.integers((32,), 10)
        model = W.CNN()
        tx, tt = torch.tensor(x), torch.tensor(t)

        def step():
            model.zero_grad()
            torch.F.cross_entropy(model(tx), tt).backward()
        sec, per, eager = _timed(torch, step, steps, warmup, graph=True)
        out.update({"metric": "small CNN fwd+bwd images/s", "value": round(32 / sec, 1),
                    "unit": "images/s", "ms_per_step": round(sec * 1e3, 3),
                    "timing": ("HIP graph replay of the whole step (hip.Graph)" if sec != eager
                               else "eager (the step could not be captured)"),
                    "eager": {"value": round(32 / eager, 1), "ms_per_step": round(eager * 1e3, 3)},
                    "roofline": {"bound": "mfma (conv2) / hbm (conv1)",
                                 "achieved": round(CNN_FLOPS / sec / 1e12, 2),
                                 "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                 "frac": round(CNN_FLOPS / sec / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4)}})
        if cpu:
            p = {k: v.numpy() for k, v in model.named_parameters()}
            dt = _cpu_time(lambda: om.cnn_loss_and_grads(p, x, t))
            out["cpu_baseline"] = {"value": round(32 / dt, 2), "unit": "images/s", "kind": "port",
                                   "sample": "oracle (numpy float64), full batch 32"}
    elif name == "block":
        r = np.random.default_rng(21)
        p = om.block_params(768, r, std=0.02)
        x = r.standard_normal((8, 1024, 768)).astype(np.float32)
        blk = W.Block(768, 12)
        W.load_params(blk, p)
        tx = torch.tensor(x, requires_grad=True)

        def step():
            blk.zero_grad()
            tx.grad = None
            blk(tx).mean().backward()
        sec, per = _timed(torch, step, steps, warmup)
        out.update({"metric": "transformer block fwd+bwd tokens/s", "value": round(8192 / sec, 1),
                    "unit": "tokens/s", "ms_per_step": round(sec * 1e3, 3),
                    "roofline": {"bound": "mfma", "achieved": round(BLOCK_FLOPS / sec / 1e12, 2),
                                 "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                 "frac": round(BLOCK_FLOPS / sec / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4),
                                 "flops": "386.58 GFLOP per step (causal-useful attention)"}})
        if cpu:
            dt = _cpu_time(lambda: om.block_loss_and_grads(p, x, 12))
            out["cpu_baseline"] = {"value": round(8192 / dt, 1), "unit": "tokens/s", "kind": "port",
                                   "sample": "oracle (numpy float64, multithreaded BLAS), full "
                                             "config: one fwd+bwd step at B=8, T=1024 (8192 "
                                             "tokens), %.1f s" % dt}
    out["kernel_ms_per_step"] = dict(list(per.items())[:10])
    if "cpu_baseline" in out:
        host = _host()
        out["cpu_baseline"]["cores"] = host["threads_used"]
        out["cpu_baseline"].update(host)
    return out


def _pmc_rows(d):
    import csv
    import glob
    rows = []
    for f in glob.glob(os.path.join(d, "*counter_collection.csv")):
        with open(f) as fh:
            rows += list(csv.DictReader(fh))
    if not rows:
        raise SystemExit("no counter_collection.csv under %s" % d)
    return rows


def summarize_pmc(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir):
    """Scales FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of the k_gemm family
    by what each counter reads for the library's copy kernel moving a known
    number of bytes, and writes the per-launch HBM bytes.  A launch is one
    GEMM call, as the library's timing counts it: its interior k_gemm
    dispatch (template flag EDGE = false) plus any guarded edge-strip
    dispatches and the split-K reduce.  Every GPT-2 product has one
    interior dispatch."""
    def is_gemm(name):
        return "k_gemm<" in name or "k_splitk_reduce" in name

    def is_copy(name):
        return "CopyOp" in name and "k_vec<1" in name

    out = {"kernel_family": "k_gemm (+ k_splitk_reduce)"}
    for cname, d, cd in (("FETCH_SIZE", fetch_dir, copy_fetch_dir),
                         ("WRITE_SIZE", write_dir, copy_write_dir)):
        copies = [float(r["Counter_Value"]) for r in _pmc_rows(cd) if is_copy(r["Kernel_Name"])]
        copy_kib = 1024.0 * 1024.0  # each calibration copy moves 1 GiB each way
        scale = copy_kib / (sum(copies) / len(copies))
        rows = [r for r in _pmc_rows(d) if is_gemm(r["Kernel_Name"])]
        launches = sum(1 for r in rows if "k_gemm<" in r["Kernel_Name"] and
                       r["Kernel_Name"].split(">")[0].endswith("false"))
        kib = sum(float(r["Counter_Value"]) for r in rows)
        out[cname] = {"raw_kib_per_launch": round(kib / launches, 1), "copy_scale": round(scale, 4),
                      "bytes_per_launch": round(kib / launches * scale * 1024.0),
                      "launches": launches}
    out["hbm_bytes_per_launch"] = out["FETCH_SIZE"]["bytes_per_launch"] + \
        out["WRITE_SIZE"]["bytes_per_launch"]
    os.makedirs(os.path.dirname(TRAFFIC_FILE), exist_ok=True)
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-workloads", action="store_true",
                    help="skip the MLP / chain / CNN / block lines of the default run")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run the copy-kernel calibration of this many MiB")
    ap.add_argument("--config", default="gpt2", choices=["gpt2"] + sorted(CONFIGS),
                    help="workload (default: the GPT-2 124M headline)")
    ap.add_argument("--summarize-pmc", nargs=4, metavar="DIR", default=None,
                    help="FETCH WRITE COPY_FETCH COPY_WRITE rocprofv3 --pmc output dirs")
    args = ap.parse_args()
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(--gpus %d requested)" % args.gpus, file=sys.stderr)
        sys.exit(2)
    if args.copy_mib:
        copy_calibration(args.copy_mib)
        return
    if args.config != "gpt2":
        print(json.dumps(run_config(args.config, args.steps, args.warmup,
                                    not args.no_cpu_baseline)), flush=True)
        return
    elapsed, final_loss, dominant, timing, prof_steps, nparams, mem, public, distinct = run_gpu(
        args.steps, args.warmup)
    tokens = B * T * args.steps
    ms_step = 1000.0 * elapsed / args.steps
    # dominant kernel: the Linear GEMMs (MFMA), timed inside the timed region
    n_g, ms_g = dominant
    flops = linear_flops_per_step(B, T) * args.steps
    achieved = flops / (ms_g / 1000.0) / 1e12 if ms_g else 0.0
    roofline = {"bound": "mfma", "kernel": "k_gemm family (Linear fwd/dgrad/wgrad + LM head, "
                "fp32 MFMA, incl. split-K reduce)",
                "achieved": round(achieved, 2), "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4), "traffic": traffic_per_launch(),
                "launches": n_g, "avg_launch_ms": round(ms_g / max(n_g, 1), 4),
                "flop_per_launch": round(flops / max(n_g, 1)),
                "share_of_step": round(ms_g / (ms_step * args.steps), 3)}
    hbm = {}
    for fam, byts in hbm_bytes_per_step(B, T, nparams, distinct).items():
        n, ms = timing.get(fam, (0, 0.0))
        if ms:
            gbs = byts * prof_steps / (ms / 1000.0) / 1e9
            hbm[fam] = {"GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 3),
                        "ms_per_step": round(ms / prof_steps, 3),
                        "launches_per_step": n // prof_steps}
    top = sorted(((ms / prof_steps, f) for f, (n, ms) in timing.items()), reverse=True)[:14]
    out = {
        "metric": METRIC, "value": round(tokens / elapsed, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic tokens uniform in [0,50257); random-init weights N(0,0.02)",
        "config": {"workload": "GPT-2 124M train step (fwd+bwd+AdamW)", "batch": B, "seq_len": T,
                   "vocab": V, "layers": LAYERS, "d_model": D, "heads": H,
                   "optimizer": "AdamW(lr=6e-4, wd=0.1)", "parallelism": "none (1 GPU)"},
        "roofline": roofline, "hbm_kernels": hbm,
        "kernel_ms_per_step": {f: round(ms, 3) for ms, f in top},
        "final_loss": round(final_loss, 4), "peak_mem_GB": round(mem["peak_bytes"] / 1e9, 2),
        "public_api": public,
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    if not args.no_workloads:
        out["workloads"] = {}
        for name in ("mlp", "chain", "cnn", "block"):
            print("workload %s" % name, file=sys.stderr, flush=True)
            out["workloads"][name] = run_config(name, WORKLOAD_STEPS[name], 3,
                                                not args.no_cpu_baseline)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
