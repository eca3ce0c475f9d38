"""Benchmark of the WKV time-mixing recurrence on one MI355X.

Default workload (one JSON line on stdout): RWKV-4 / SpikeGPT WKV forward +
backward, bf16 I/O with fp32 state, B=64, T=1024, C=512 -- the 41M SpikeGPT
training shape.  A "step" is one forward + backward pass of the recurrence over one batch
that is already resident in HBM.

The timed region issues that step through the C ABI on buffers allocated
once (``wkv4_forward_checkpointed`` then ``wkv4_backward_checkpointed``, the
two launches the autograd path makes), so the number is the kernels' own
throughput; the same work through the Python API the reference's time mix
calls (``weighted_key_value_triton_bf16io``: dispatch, allocation and
autograd on every call) is reported as ``op_ms_per_step``, as
``op_ms_per_step_backward_on_calling_thread`` with the autograd engine's
per-device worker threads switched off
(``torch.autograd.set_multithreading_enabled(False)``), which removes the
engine's hand-off of every backward to its device thread, and through the
public op ``myelin::wkv_forward_bf16io`` called directly (its autograd saves
only the inputs and its backward recomputes the forward's records, as the
reference's does) as ``public_op_ms_per_step``.

Reported beside the throughput:
* ``roofline`` -- the dominant kernel (the backward's reverse sweep,
  ``wkv4_bwd_kernel``, or ``wkv4_bwd_split_kernel`` for few rows), timed
  alone on every 10th step of the timed region (``--event-every``) with HIP
  events bound to its own dispatch (``wkv_time_next_kernel``: the kernel's
  start and end timestamps on the launch stream, no marker packets);
  algorithmic bytes = 10 B per [B,T,C] element (k, v, dy read, dk, dv
  written); peak 8 TB/s.  ``traffic`` comes from the committed rocprofv3 PMC
  summary of that kernel (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the
  same counters on a copy of known size) when present, else null.
* ``cpu_baseline`` -- the reference's CPU WKV path restated in eager PyTorch
  (the sequential loop of src/spikegpt/language.py:399-449 in fp32, backward
  by autograd) on a bounded sample of the same workload, on this host's cores.

Other workloads (``--workload``): ``long`` (B=24, T=3072, C=512), ``216m``
(B=16, T=1024, C=768, 18 layers), ``decode`` (B=256, C=768, 18 layers, fp32
state), ``wkv7`` (RWKV-7 B=16, T=1024, H=12, N=64 forward + backward), ``c0``
(fp32 forward B=2, T=128, C=512), ``block_decode`` (whole 216M model one-token
decode, B=256, fused block step in one HIP graph), ``lif`` (sequence LIF forward + backward, B=64, T=1024, C=512 bf16),
``timemix`` (fused token-shift mix, three vectors, same shape),
``e2e41m`` (the whole 41M SpikeGPT
training step, 12 layers x 512, vocab 256, B=64, T=1024; the default run
also reports it as ``e2e_train_step``), ``e2e216m`` (the 216M-class training
step, 18 layers x 768, vocab 50277, B=16, T=1024).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
HBM_PEAK_GBS = 8000.0
FP32_VALU_PEAK_TFLOPS = 157.3
METRIC = "WKV fwd+bwd tokens/sec & HBM GB/s (% of peak), B=64 T=1024 C=512 bf16"

WORKLOADS = {
    "wkv4": dict(B=64, T=1024, C=512, dtype=torch.bfloat16, layers=1, slug="wkv4_b64_t1024_c512"),
    "long": dict(B=24, T=3072, C=512, dtype=torch.bfloat16, layers=1, slug="wkv4_b24_t3072_c512"),
    "216m": dict(B=16, T=1024, C=768, dtype=torch.bfloat16, layers=18,
                 slug="wkv4_b16_t1024_c768_x18"),
    "c0": dict(B=2, T=128, C=512, dtype=torch.float32, layers=1, slug="wkv4_fwd_f32_b2_t128_c512"),
}


def settle_gc() -> None:
    """Collects, then moves every object alive now into the collector's
    permanent generation (``gc.freeze``), so that a later full collection
    scans only the objects made after this point.  Called before each timed
    region: a full collection in a process holding torch's modules takes tens
    of milliseconds, and one that fell inside a timed region of a host-bound
    route (the op paths, ~0.2 ms of Python per step) added that to the
    region (the public-op route read 0.59 against 0.19 ms per step)."""
    gc.collect()
    gc.freeze()


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def keep_heap_for_large_blocks() -> bool:
    """Serve allocations up to 256 MiB from glibc's heap and keep freed heap
    memory in the process (``mallopt(M_MMAP_THRESHOLD)``,
    ``mallopt(M_TRIM_THRESHOLD)``).

    The reference loop's autograd backward builds a full ``[B, T, C]`` zero
    tensor for the gradient of every ``key[:, t]`` / ``value[:, t]`` slice
    (32 MiB each at the B=16 sample, above glibc's largest dynamic mmap
    threshold), so by default every one is a fresh mmap whose pages fault in
    on first touch: ~12.6 million minor faults per run, and a run time set by
    the host kernel's page-fault throughput (3.3e3 to 2.1e4 tokens/s from run
    to run on one host).  With the heap kept, the same runs take ~1e3x fewer
    faults and repeat within a few percent.  Returns False where the C
    library has no ``mallopt`` (the figure then includes the faults)."""
    import ctypes

    try:
        libc = ctypes.CDLL("libc.so.6")
        m_trim_threshold, m_mmap_threshold = -1, -3
        return bool(libc.mallopt(m_mmap_threshold, 256 << 20)
                    and libc.mallopt(m_trim_threshold, 1 << 30))
    except (OSError, AttributeError):
        return False


def timed_cpu_runs(once, min_runs: int = 5, max_runs: int = 15, budget_s: float = 12.0) -> dict:
    """Run ``once`` fully once (warm-up: allocator, autograd graph, thread
    pool), then at least ``min_runs`` and at most ``max_runs`` timed times,
    stopping after ``budget_s`` seconds once ``min_runs`` are done.  Returns
    the fastest, median and slowest run, the minor page faults per timed run
    and the host's load average before and after (other tenants' load on the
    host's cores slows single runs; the fastest run is the least disturbed
    one)."""
    import resource

    heap_kept = keep_heap_for_large_blocks()
    load_before = os.getloadavg()
    once()
    settle_gc()
    times = []
    faults0 = resource.getrusage(resource.RUSAGE_SELF).ru_minflt
    start = time.perf_counter()
    while len(times) < max_runs and (len(times) < min_runs
                                     or time.perf_counter() - start < budget_s):
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
    faults = resource.getrusage(resource.RUSAGE_SELF).ru_minflt - faults0
    return {"min_s": min(times), "median_s": statistics.median(times), "max_s": max(times),
            "runs": len(times), "loadavg_before": [round(x, 2) for x in load_before],
            "loadavg_after": [round(x, 2) for x in os.getloadavg()],
            "minor_faults_per_run": faults // len(times), "heap_kept": heap_kept}


def cpu_baseline(B: int, T: int, C: int, sample_batch: int, fwd_only: bool = False) -> dict:
    """The reference CPU path (eager loop, fp32, autograd) on a batch sample.

    ``value`` is the fastest of the timed runs; the median and slowest runs,
    the thread count and the host's load average are reported beside it."""
    sys.path.insert(0, str(ROOT))
    from oracle import wkv4 as O

    torch.set_num_threads(os.cpu_count() or 1)
    bs = min(B, sample_batch)
    k, v, td, tf, dy = O.make_inputs(bs, T, C, seed=0, dtype=torch.bfloat16)
    k, v, dy = k.float(), v.float(), dy.float()  # the reference upcasts (language.py:483-485)

    def once():
        if fwd_only:
            with torch.no_grad():
                O.wkv_loop(k, v, td, tf)
            return
        leaves = [x.clone().requires_grad_(True) for x in (k, v, td, tf)]
        y = O.wkv_loop(*leaves)
        torch.autograd.grad(y, leaves, dy)

    r = timed_cpu_runs(once)
    out = {
        "value": bs * T / r["min_s"],
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"B={bs} of {B}, T={T}, C={C}, fp32 eager loop "
                   f"{'forward' if fwd_only else 'forward+autograd backward'}, "
                   f"fastest of {r['runs']} runs after 1 full warm-up run"
                   f"{', glibc heap kept for blocks up to 256 MiB' if r['heap_kept'] else ''}; "
                   f"torch.get_num_threads()={torch.get_num_threads()}; host {_cpu_model()}, "
                   f"os.cpu_count()={os.cpu_count()}"),
        "median_value": bs * T / r["median_s"],
        "slowest_value": bs * T / r["max_s"],
        "runs": r["runs"],
        "loadavg_before": r["loadavg_before"],
        "loadavg_after": r["loadavg_after"],
        "minor_faults_per_run": r["minor_faults_per_run"],
        "heap_kept": r["heap_kept"],
    }
    out["secondary"] = associative_scan_baseline(B, T, C)
    return out


def associative_scan_baseline(B: int, T: int, C: int, sample_batch: int = 64) -> dict:
    """The reference's default CPU path, ``weighted_key_value``
    (src/spikegpt/language.py:452-527: torch associative_scan over the
    log-space monoid, generic combine mode), forward only, fp32."""
    from oracle import wkv4 as O

    bs = min(B, sample_batch)
    k, v, td, tf, _ = O.make_inputs(bs, T, C, seed=0, dtype=torch.bfloat16)
    k, v = k.float(), v.float()
    def once():
        with torch.no_grad():
            O.wkv_associative_scan(k, v, td, tf)

    r = timed_cpu_runs(once, budget_s=6.0)
    return {
        "value": bs * T / r["min_s"],
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"B={bs} of {B}, T={T}, C={C}, fp32, torch associative_scan (generic "
                   f"combine) forward only, fastest of {r['runs']} runs after 1 warm-up run; "
                   "autograd unverified on torch < 2.13 (this image: torch "
                   + torch.__version__.split("+")[0] + ")"),
        "median_value": bs * T / r["median_s"],
        "slowest_value": bs * T / r["max_s"],
        "runs": r["runs"],
    }


def read_traffic(path: Path, kernel: str) -> int | None:
    """HBM bytes per dispatch of ``kernel`` from a committed PMC summary of the
    same workload.

    The summary lists ``traffic_bytes <kernel> <N>`` lines (FETCH_SIZE +
    WRITE_SIZE scaled by a copy-kernel calibration)."""
    if not path.exists():
        return None
    m = re.search(rf"^traffic_bytes\s+{re.escape(kernel)}\s+(\d+)", path.read_text(), re.M)
    return int(m.group(1)) if m else None


def event_offset(args) -> int:
    """Step (mod --event-every) whose launches carry the timing events: the
    middle of the first block of steps, not the timed region's first step
    (which follows a synchronisation), as long as the region has it."""
    return min(args.event_every // 2, max(args.steps - 1, 0))


class EventPool:
    """Timing events created and recorded once before the timed region (a
    HIP event is created at its first record, which costs host time that
    would otherwise land inside the timed loop)."""

    def __init__(self, n: int, stream) -> None:
        self.events = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
        for ev in self.events:
            ev.record(stream)
        torch.cuda.synchronize()
        self.next = 0

    def take(self):
        ev = self.events[self.next]
        self.next += 1
        return ev

    def reset(self) -> None:
        self.next = 0


def bench_wkv4(args, cfg) -> dict:
    import spikegpt_myelin_amd  # noqa: F401  -- registers the ops
    from spikegpt_myelin_amd import _lib
    from spikegpt_myelin_amd.wkv import checkpoint_shape
    from oracle import wkv4 as O

    B, T, C, dtype, layers = cfg["B"], cfg["T"], cfg["C"], cfg["dtype"], cfg["layers"]
    dev = torch.device("cuda", 0)
    k, v, td, tf, dy = (x.to(dev) for x in O.make_inputs(B, T, C, seed=1, dtype=dtype))
    fwd_only = args.workload == "c0"
    lib = _lib.load()
    code = _lib.dtype_code(dtype)
    # Outputs and scratch allocated once: the timed region is the kernels.
    y = torch.empty_like(k)
    ck = torch.empty(checkpoint_shape(B, T, C), dtype=torch.float32, device=dev)
    gk, gv = torch.empty_like(k), torch.empty_like(k)
    gtd = torch.empty(C, dtype=torch.float32, device=dev)
    gtf = torch.empty(C, dtype=torch.float32, device=dev)
    # Workspaces: the split-over-time kernels' carries (few rows) and the
    # backward's parameter-gradient partials.
    fws_bytes = int(lib.wkv4_forward_workspace_bytes(B, T, C))
    fws = torch.empty(max(fws_bytes, 16), dtype=torch.uint8, device=dev)
    bws_bytes = int(lib.wkv4_backward_checkpointed_workspace_bytes(B, T, C))
    ws = torch.empty(bws_bytes, dtype=torch.uint8, device=dev)
    split = fws_bytes > 0
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream

    def fwd():
        _lib.check(lib.wkv4_forward_checkpointed(k.data_ptr(), v.data_ptr(), td.data_ptr(),
                                                 tf.data_ptr(), y.data_ptr(), ck.data_ptr(),
                                                 fws.data_ptr() if split else None, fws_bytes,
                                                 B, T, C, code, sp), "forward")

    def bwd():
        _lib.check(lib.wkv4_backward_checkpointed(dy.data_ptr(), td.data_ptr(), tf.data_ptr(),
                                                  k.data_ptr(), v.data_ptr(), ck.data_ptr(),
                                                  gk.data_ptr(), gv.data_ptr(), gtd.data_ptr(),
                                                  gtf.data_ptr(), ws.data_ptr(), bws_bytes,
                                                  B, T, C, code, sp), "backward")

    # The same work through the drop-in entry points (dispatch, allocation and
    # autograd on every call), for reference; timed first, in a process with
    # no timing events outstanding.  `api`: the Python API the reference's
    # SpikeTimeMix calls (weighted_key_value_triton{,_bf16io}), whose backward
    # reads the forward's records; `public_op`: the public torch.library op
    # called directly, whose autograd saves only the inputs and whose backward
    # op computes the records again, as the reference's does.
    from spikegpt_myelin_amd import weighted_key_value_triton, weighted_key_value_triton_bf16io

    leaves = [x.detach().requires_grad_(True) for x in (k, v, td, tf)]
    routes = {
        "api": weighted_key_value_triton_bf16io if dtype != torch.float32
        else weighted_key_value_triton,
        "public_op": torch.ops.myelin.wkv_forward_bf16io if dtype != torch.float32
        else torch.ops.myelin.wkv_forward,
    }

    def time_op_path(fwd_op):
        def op_step():
            for _ in range(layers):
                if fwd_only:
                    with torch.no_grad():
                        fwd_op(*leaves)
                else:
                    torch.autograd.grad(fwd_op(*leaves), leaves, dy)

        for _ in range(args.warmup):
            op_step()
        torch.cuda.synchronize()
        settle_gc()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            op_step()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / args.steps

    op_step_s = time_op_path(routes["api"])
    public_op_step_s = time_op_path(routes["public_op"])
    # The same with the autograd engine running the backward on the calling
    # thread (no hand-off to its per-device worker thread).
    with torch.autograd.set_multithreading_enabled(False):
        op_step_1t_s = time_op_path(routes["api"])

    dom_name = "fwd" if fwd_only else "bwd"
    # The dominant kernel: the reverse sweep of the backward (the forward for
    # a forward-only workload), the launch's first dispatch, or its second
    # after the fill of the split kernels' carry words.
    dom_index = 1 if split else 0
    pool = EventPool(4 * args.steps * layers, stream)

    def step(events=None, timed=(dom_name,), kernel=None):
        # The launches named in `timed` carry HIP events on their first and
        # last kernel dispatch, or on their `kernel`-th dispatch alone (kernel
        # start/end timestamps; the stream gets no marker packets, so the
        # timed step is not perturbed).
        for _ in range(layers):
            for name, fn in (("fwd", fwd),) if fwd_only else (("fwd", fwd), ("bwd", bwd)):
                if events is None or name not in timed:
                    fn()
                    continue
                s_ev = pool.take()
                e_ev = pool.take()
                _lib.arm_events(s_ev, e_ev, kernel)
                fn()
                events.append((name, s_ev, e_ev))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    settle_gc()
    # Timed region: K steps; events around the dominant launch only.
    events: list = []
    t0 = time.perf_counter()
    for i in range(args.steps):
        # Every `event_every`-th step carries the events (from the middle of
        # the first block on, not the region's first step, which follows the
        # synchronisation), so the other steps run undisturbed.
        timed_step = i % args.event_every == event_offset(args)
        step(events if timed_step else None, kernel=dom_index)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    step_s = elapsed / args.steps
    per = {}
    for name, s_ev, e_ev in events:
        per.setdefault(name, []).append(s_ev.elapsed_time(e_ev) * 1e-3)
    # Check pass (not in `value`): the dominant dispatch timed on every one of
    # at least 100 steps, the same binding as above.
    check_steps = max(100, args.steps)
    if 2 * check_steps * layers > len(pool.events):
        pool = EventPool(2 * check_steps * layers, stream)
    pool.reset()
    events = []
    for _ in range(check_steps):
        step(events, kernel=dom_index)
    torch.cuda.synchronize()
    check = [s_ev.elapsed_time(e_ev) * 1e-3 for name, s_ev, e_ev in events if name == dom_name]
    # Attribution pass (not in `value`): events around every launch.
    pool.reset()
    events = []
    for _ in range(args.steps):
        step(events, timed=("fwd", "bwd"))
    torch.cuda.synchronize()
    attr = {}
    for name, s_ev, e_ev in events:
        attr.setdefault(name, []).append(s_ev.elapsed_time(e_ev) * 1e-3)
    fwd_s = statistics.mean(attr["fwd"])
    bwd_s = statistics.mean(attr["bwd"]) if "bwd" in attr else float("nan")


    esize = torch.finfo(dtype).bits // 8
    n_elem = B * T * C * layers
    tokens = B * T * args.steps
    alg_step = (3 * esize if fwd_only else 8 * esize) * n_elem  # fwd k,v,y; bwd k,v,dy,dk,dv
    out = {
        "metric": METRIC if args.workload == "wkv4" else f"WKV {'fwd' if fwd_only else 'fwd+bwd'} tokens/sec "
                                                        f"B={B} T={T} C={C} x{layers} layers",
        "value": tokens / elapsed,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"wkv4_{'fwd' if fwd_only else 'fwd_bwd'}", "B": B, "T": T, "C": C,
                   "layers": layers, "io_dtype": str(dtype).replace("torch.", ""),
                   "state_dtype": "float32", "parallelism": "single_gpu",
                   "timing": "C-ABI launches on preallocated buffers (op path in op_ms_per_step)"},
        "hbm_gbps_algorithmic": alg_step / step_s / 1e9,
        "hbm_frac_of_peak": alg_step / step_s / 1e9 / HBM_PEAK_GBS,
        "op_ms_per_step": op_step_s * 1e3,
        "op_tokens_per_s": B * T / op_step_s,
        "op_ms_per_step_backward_on_calling_thread": op_step_1t_s * 1e3,
        "public_op_ms_per_step": public_op_step_s * 1e3,
        "fwd_launch_us": fwd_s * 1e6,
    }
    dom_t = statistics.mean(per[dom_name])
    if fwd_only:
        dom = "wkv4_fwd_split_kernel" if split else "wkv4_fwd_kernel"
        dom_bytes = 3 * esize * B * T * C
        entry = "wkv4_forward_checkpointed"
    else:
        out["bwd_launch_us"] = bwd_s * 1e6
        dom = "wkv4_bwd_split_kernel" if split else "wkv4_bwd_kernel"
        dom_bytes = 5 * esize * B * T * C
        entry = "wkv4_backward_checkpointed"
    achieved = dom_bytes / dom_t / 1e9
    traffic_file = ROOT / "profiles" / f"{cfg['slug']}_pmc.md"
    traffic = read_traffic(traffic_file, dom)
    out["roofline"] = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                       "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "kernel": dom,
                       "algorithmic_bytes_per_launch": dom_bytes,
                       "avg_launch_us": dom_t * 1e6,
                       "samples": len(per[dom_name]),
                       "check_avg_launch_us": statistics.mean(check) * 1e6,
                       "check_median_launch_us": statistics.median(check) * 1e6,
                       "check_samples": len(check),
                       "launch": f"{entry}, dispatch {dom_index} ({dom}) timed alone",
                       "traffic_source": (str(traffic_file.relative_to(ROOT))
                                          if traffic is not None else None)}
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(B, T, C, args.cpu_sample_batch, fwd_only=fwd_only)
    return out


def bench_decode(args) -> dict:
    import spikegpt_myelin_amd  # noqa: F401
    from spikegpt_myelin_amd import _lib, initial_wkv_state
    from oracle import wkv4 as O

    B, C, layers = 256, 768, 18
    dev = torch.device("cuda", 0)
    ks, vs, tds, tfs = [], [], [], []
    for layer in range(layers):
        k, v, td, tf, _ = O.make_inputs(B, 1, C, seed=100 + layer, with_grad=False)
        ks.append(k[:, 0].to(dev)); vs.append(v[:, 0].to(dev)); tds.append(td.to(dev)); tfs.append(tf.to(dev))
    states = [initial_wkv_state(B, C, dev) for _ in range(layers)]
    ys = [torch.empty_like(k) for k in ks]
    lib = _lib.load()
    code = _lib.dtype_code(torch.float32)

    def step():
        # One token through the 18 layers' state updates (C-ABI launches on
        # the current stream, state updated in place, outputs preallocated).
        sp = torch.cuda.current_stream(dev).cuda_stream
        for layer in range(layers):
            num, den, ls = states[layer]
            _lib.check(lib.wkv4_decode_step(
                ks[layer].data_ptr(), vs[layer].data_ptr(), tds[layer].data_ptr(),
                tfs[layer].data_ptr(), num.data_ptr(), den.data_ptr(), ls.data_ptr(),
                ys[layer].data_ptr(), num.data_ptr(), den.data_ptr(), ls.data_ptr(), B, C, code, sp),
                "decode")

    def timed(fn) -> float:
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        settle_gc()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            fn()
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    eager = timed(step)
    # The same 18 launches captured once in a HIP graph and replayed per token
    # (what a generation loop does: see spikegpt_myelin_amd.generation).
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream(dev).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    elapsed = timed(graph.replay)
    per_layer = elapsed / args.steps / layers
    alg = 36 * B * C  # k, v read (8 B); state read and written (24 B); y written (4 B)
    achieved = alg / per_layer / 1e9
    out = {
        "metric": "WKV decode state update tokens/sec, B=256 C=768 x18 layers fp32 state",
        "value": B * args.steps / elapsed, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": elapsed / args.steps * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "wkv4_decode_step", "B": B, "C": C, "layers": layers,
                   "launch": "18 launches per token captured in one HIP graph"},
        "us_per_layer_step": per_layer * 1e6,
        "eager_us_per_layer_step": eager / args.steps / layers * 1e6,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "kernel": "wkv4_decode_kernel (per-layer graph time, dispatch gaps included)",
                     "algorithmic_bytes_per_launch": alg},
    }
    if not args.no_cpu_baseline:
        # The reference's decode is this eager step (language.py:989-1012),
        # restated by the oracle: one token through the 18 layers on the host.
        torch.set_num_threads(os.cpu_count() or 1)
        kc = [k.cpu() for k in ks]
        vc = [v.cpu() for v in vs]
        tdc = [t.cpu() for t in tds]
        tfc = [t.cpu() for t in tfs]
        cst = [O.initial_decode_state(B, C) for _ in range(layers)]

        def cpu_token():
            for layer in range(layers):
                _, *cst[layer] = O.decode_step(kc[layer], vc[layer], tdc[layer], tfc[layer],
                                               *cst[layer])

        cpu_token()
        n = 50
        t0 = time.perf_counter()
        for _ in range(n):
            cpu_token()
        dt = time.perf_counter() - t0
        out["cpu_baseline"] = {
            "value": B * n / dt, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{n} tokens at B={B}, C={C} through the {layers} layers' WKV state "
                      f"updates, the oracle's eager fp32 step (language.py:989-1012 restated); "
                      f"host {_cpu_model()}"}
    return out


def bench_block_decode(args) -> dict:
    """Whole-model one-token decode of the 216M SpikeGPT (18 layers x 768,
    BPE vocab 50277, fp32 weights and state) at batch 256: the fused block-step
    kernels and the projections, captured in one HIP graph per token
    (spikegpt_myelin_amd.generation.StepGraph), random init, synthetic ids."""
    from spikegpt_myelin_amd.generation import StepGraph
    from spikegpt_myelin_amd.model import SpikeGPTConfig, SpikeLanguageModel

    B, C, layers, vocab = 256, 768, 18, 50277
    dev = torch.device("cuda", 0)
    torch.manual_seed(0)
    cfg = SpikeGPTConfig(vocab_size=vocab, context_length=1024, n_layer=layers, n_embd=C,
                         dropout=0.0)
    model = SpikeLanguageModel(cfg).to(dev).eval()
    graph = StepGraph(model, B)
    gen = torch.Generator(device=dev).manual_seed(1)
    ids = torch.randint(0, vocab, (args.steps + args.warmup, B), device=dev, generator=gen)
    for i in range(args.warmup):
        graph.step(ids[i])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    settle_gc()
    t0 = time.perf_counter()
    e0.record()
    for i in range(args.steps):
        graph.step(ids[args.warmup + i])
    e1.record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    step_s = e0.elapsed_time(e1) / 1e3 / args.steps
    # Multiply-accumulates per token: 13 C^2 per layer (k, v, r, output,
    # receptance: C^2 each; key and value: 4 C^2 each) plus the head.
    macs = layers * 13 * C * C + C * vocab
    flops = 2.0 * B * macs
    out = {
        "metric": "SpikeGPT-216M one-token decode tokens/sec (whole model, fused block step, "
                  "HIP graph), B=256 fp32",
        "value": B * args.steps / elapsed, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": elapsed / args.steps * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "block_decode_216m", "B": B, "C": C, "layers": layers,
                   "vocab": vocab, "params": sum(p.numel() for p in model.parameters())},
        "roofline": {"bound": "mfma", "achieved": flops / step_s / 1e12, "peak": 157.3,
                     "unit": "TFLOP/s", "frac": flops / step_s / 1e12 / 157.3, "traffic": None,
                     "kernel": "whole step (fp32 projections dominate), HIP-event timed"},
    }
    if not args.no_cpu_baseline:
        from oracle import step as S

        sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
        sc = S.StepConfig.of(cfg)
        cb = max(1, min(B, args.cpu_sample_batch * 4))
        state = S.initial_state(sc, cb)
        cids = ids[:, :cb].cpu()
        n = 4
        S.model_forward_step(sd, sc, cids[0], state)
        t0 = time.perf_counter()
        for i in range(n):
            _, state = S.model_forward_step(sd, sc, cids[i + 1], state)
        dt = time.perf_counter() - t0
        out["cpu_baseline"] = {
            "value": cb * n / dt, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{n} tokens at batch {cb} through the oracle's eager fp32 step of the "
                      f"same model (language.py:1434-1453 restated), torch CPU"}
    return out


def bench_wkv7(args) -> dict:
    """RWKV-7 DPLR forward (with state checkpoints) + backward through the C
    ABI on preallocated buffers, B=16 T=1024 H=12 N=64, bf16 I/O, fp32 state."""
    import spikegpt_myelin_amd  # noqa: F401
    from spikegpt_myelin_amd import _lib
    from spikegpt_myelin_amd.wkv7 import checkpoint_shape
    from oracle import wkv7 as O7

    B, T, H, N = 16, 1024, 12, 64
    dev = torch.device("cuda", 0)
    xs = [x.to(dev) for x in O7.make_inputs(B, T, H, N, seed=4, dtype=torch.bfloat16)]
    gy = torch.randn(B, T, H, N, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(dev)
    y = torch.empty_like(xs[0])
    s_out = torch.empty(B, H, N, N, dtype=torch.float32, device=dev)
    ck = torch.empty(checkpoint_shape(B, T, H), dtype=torch.float32, device=dev)
    grads = [torch.empty_like(xs[0]) for _ in range(6)]
    lib = _lib.load()
    code = _lib.dtype_code(torch.bfloat16)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    ptrs = [x.data_ptr() for x in xs]

    def fwd():
        _lib.check(lib.wkv7_forward_checkpointed(*ptrs, None, y.data_ptr(), s_out.data_ptr(),
                                                 ck.data_ptr(), B, T, H, N, code, sp), "wkv7 forward")

    def bwd():
        _lib.check(lib.wkv7_backward_checkpointed(*ptrs, ck.data_ptr(), gy.data_ptr(), None,
                                                  *[g.data_ptr() for g in grads], None,
                                                  B, T, H, N, code, sp), "wkv7 backward")

    pool = EventPool(4 * args.steps, stream)
    for _ in range(args.warmup):
        fwd()
        bwd()
    torch.cuda.synchronize()
    settle_gc()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        fwd()
        bwd()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    step_s = elapsed / args.steps
    per = {"fwd": [], "bwd": []}
    evs = []
    for _ in range(args.steps):
        for name, fn in (("fwd", fwd), ("bwd", bwd)):
            s_ev, e_ev = pool.take(), pool.take()
            _lib.arm_events(s_ev, e_ev)
            fn()
            evs.append((name, s_ev, e_ev))
    torch.cuda.synchronize()
    for name, s_ev, e_ev in evs:
        per[name].append(s_ev.elapsed_time(e_ev) * 1e-3)
    fwd_t, bwd_t = statistics.mean(per["fwd"]), statistics.mean(per["bwd"])
    units = B * T * H
    fwd_flops = 9 * N * N * units   # sa, update, y per state element
    bwd_flops = 19 * N * N * units  # reverse recurrence (recomputation not counted)
    fwd_bytes = 14 * N * units      # r, w, k, v, a, b read, y written (bf16)
    bwd_bytes = 26 * N * units      # 6 inputs + dy read, 6 grads written (bf16)
    achieved = bwd_flops / bwd_t / 1e12
    out = {
        "metric": "RWKV-7 DPLR fwd+bwd tokens/sec, B=16 T=1024 H=12 N=64 bf16 I/O fp32 state",
        "value": B * T / step_s, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": step_s * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "wkv7_fwd_bwd", "B": B, "T": T, "H": H, "N": N,
                   "io_dtype": "bfloat16", "state_dtype": "float32",
                   "timing": "C-ABI launches on preallocated buffers"},
        "fwd_launch_us": fwd_t * 1e6, "bwd_launch_us": bwd_t * 1e6,
        "fwd_tflops": fwd_flops / fwd_t / 1e12,
        "hbm_gbps_algorithmic": (fwd_bytes + bwd_bytes) / step_s / 1e9,
        "roofline": {"bound": "valu", "achieved": achieved, "peak": FP32_VALU_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / FP32_VALU_PEAK_TFLOPS, "traffic": None,
                     "kernel": "wkv7_bwd_kernel", "algorithmic_flops_per_launch": bwd_flops,
                     "avg_launch_us": bwd_t * 1e6},
    }
    if not args.no_cpu_baseline:
        # No CPU path survives in the reference for RWKV-7 (its code was
        # deleted); the oracle's fp32 loops are the host counterpart: the
        # forward recurrence, then the explicit reverse recurrence.
        torch.set_num_threads(os.cpu_count() or 1)
        bs = 1
        xc = [x[:bs].float().cpu() for x in xs]
        gyc = gy[:bs].float().cpu()
        t0 = time.perf_counter()
        O7.wkv7_loop(*xc)
        O7.wkv7_backward_loop(*xc, None, gyc)
        dt = time.perf_counter() - t0
        out["cpu_baseline"] = {
            "value": bs * T / dt, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"B={bs} of {B}, T={T}, H={H}: the oracle's fp32 forward loop and explicit "
                      f"reverse loop (the reference's RWKV-7 code was deleted), one run; host "
                      f"{_cpu_model()}"}
    return out


def bench_lif(args) -> dict:
    """Sequence LIF forward (with membrane checkpoints) + backward through the
    C ABI on preallocated buffers: B=64, T=1024, C=512 bf16 (the 41M model's
    activation shape), tau 2, threshold 1, reset 0, slope 2."""
    import spikegpt_myelin_amd  # noqa: F401
    from spikegpt_myelin_amd import _lib
    from spikegpt_myelin_amd.lif import checkpoint_shape
    from oracle import lif as L

    B, T, C = 64, 1024, 512
    decay, thr, reset, slope = 0.5, 1.0, 0.0, 2.0
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(B, T, C, generator=g).to(torch.bfloat16).to(dev)
    gs = torch.randn(B, T, C, generator=g).to(torch.bfloat16).to(dev)
    spk = torch.empty_like(x)
    gx = torch.empty_like(x)
    ck = torch.empty(checkpoint_shape(B, T, C), dtype=torch.float32, device=dev)
    lib = _lib.load()
    code = _lib.dtype_code(torch.bfloat16)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    ws_bytes = int(lib.lif_forward_workspace_bytes(B, T, C))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    bws_bytes = int(lib.lif_backward_workspace_bytes(B, T, C))
    bws = torch.empty(max(bws_bytes, 16), dtype=torch.uint8, device=dev)
    xp, spkp, ckp, gsp, gxp, wsp, bwsp = (t.data_ptr() for t in (x, spk, ck, gs, gx, ws, bws))

    def fwd():
        _lib.check(lib.lif_forward(xp, spkp, ckp, wsp, ws_bytes, B, T, C, decay, thr, reset, slope,
                                   code, sp), "lif forward")

    def bwd():
        _lib.check(lib.lif_backward(xp, gsp, ckp, gxp, bwsp, bws_bytes, B, T, C, decay, thr, reset,
                                    slope, code, sp), "lif backward")

    pool = EventPool(4 * args.steps, stream)
    for _ in range(args.warmup):
        fwd()
        bwd()
    torch.cuda.synchronize()
    evs, fevs = [], []
    settle_gc()
    t0 = time.perf_counter()
    for i in range(args.steps):
        if i % args.event_every == event_offset(args):
            s_ev, e_ev = pool.take(), pool.take()
            _lib.arm_events(s_ev, e_ev)
            fwd()
            fevs.append((s_ev, e_ev))
            s_ev, e_ev = pool.take(), pool.take()
            _lib.arm_events(s_ev, e_ev)
            bwd()
            evs.append((s_ev, e_ev))
        else:
            fwd()
            bwd()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    bwd_t = statistics.mean(s.elapsed_time(e) * 1e-3 for s, e in evs)
    fwd_t = statistics.mean(s.elapsed_time(e) * 1e-3 for s, e in fevs)
    step_s = elapsed / args.steps
    n = B * T * C
    bwd_bytes = 6 * n  # x, grad_spikes read; grad_x written (bf16)
    achieved = bwd_bytes / bwd_t / 1e9
    out = {
        "metric": "sequence LIF fwd+bwd tokens/sec, B=64 T=1024 C=512 bf16",
        "value": B * T / step_s, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": step_s * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "lif_fwd_bwd", "B": B, "T": T, "C": C, "io_dtype": "bfloat16",
                   "state_dtype": "float32", "tau": 2.0, "threshold": thr, "reset": reset,
                   "slope": slope},
        "hbm_gbps_algorithmic": 10 * n / step_s / 1e9,
        "fwd_launch_us": fwd_t * 1e6, "bwd_launch_us": bwd_t * 1e6,
        "fwd_gbps_algorithmic": 4 * n / fwd_t / 1e9,
        "fwd_time_segments": int(ws_bytes // (8 * B * C)) + 1 if ws_bytes else 1,
        "bwd_time_segments": int(bws_bytes // (8 * B * C)) + 1 if bws_bytes else 1,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel": "lif_bwd_kernel",
                     "algorithmic_bytes_per_launch": bwd_bytes, "avg_launch_us": bwd_t * 1e6},
    }
    if not args.no_cpu_baseline:
        torch.set_num_threads(os.cpu_count() or 1)
        bs = min(B, args.cpu_sample_batch)
        xc = x[:bs].float().cpu().requires_grad_(True)
        gc = gs[:bs].float().cpu()
        times = []
        for _ in range(3):
            t1 = time.perf_counter()
            torch.autograd.grad(L.lif_loop(xc), xc, gc)
            times.append(time.perf_counter() - t1)
        med = statistics.median(times[1:])
        out["cpu_baseline"] = {
            "value": bs * T / med, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"B={bs} of {B}, T={T}, C={C}, fp32 eager LIF loop (language.py:813-840, "
                       f"908-918) forward+autograd backward, median of 2 after 1 warmup; host "
                       f"{_cpu_model()}"),
        }
    return out


def bench_gated(args) -> dict:
    """The time mix's WKV with its receptance gate, ``sigmoid(r) * wkv``
    (src/spikegpt/language.py:1028-1035), forward + backward at B=64,
    T=1024, C=512 bf16, two ways through the C ABI on preallocated buffers,
    timed back to back in one process:
    * fused: ``wkv4_forward_gated_checkpointed`` then
      ``wkv4_backward_gated_checkpointed`` (the gate inside the WKV kernels);
    * unfused: ``wkv4_forward_checkpointed``, ``sigmoid_gate_forward``, then
      ``sigmoid_gate_backward`` and ``wkv4_backward_checkpointed``.
    Both give the same values bit for bit (tests/test_gpu_wkv4_gated.py).
    ``value`` is the variant the model uses (``config.model_uses``)."""
    import spikegpt_myelin_amd  # noqa: F401
    from spikegpt_myelin_amd import _lib
    from spikegpt_myelin_amd.wkv import GATED_TIME_MIX, checkpoint_shape
    from oracle import wkv4 as O

    B, T, C = 64, 1024, 512
    dt = torch.bfloat16
    dev = torch.device("cuda", 0)
    k, v, td, tf, dy = (x.to(dev) for x in O.make_inputs(B, T, C, seed=1, dtype=dt))
    r = (torch.randn(B, T, C, generator=torch.Generator().manual_seed(9)) * 2).to(dt).to(dev)
    lib = _lib.load()
    code = _lib.dtype_code(dt)
    y, out = torch.empty_like(k), torch.empty_like(k)
    ck = torch.empty(checkpoint_shape(B, T, C), dtype=torch.float32, device=dev)
    gk, gv, gr, gy = (torch.empty_like(k) for _ in range(4))
    gtd = torch.empty(C, dtype=torch.float32, device=dev)
    gtf = torch.empty_like(gtd)
    fws_bytes = int(lib.wkv4_forward_workspace_bytes(B, T, C))
    fws = torch.empty(max(fws_bytes, 16), dtype=torch.uint8, device=dev)
    bws_bytes = int(lib.wkv4_backward_checkpointed_workspace_bytes(B, T, C))
    ws = torch.empty(bws_bytes, dtype=torch.uint8, device=dev)
    fwp = fws.data_ptr() if fws_bytes else None
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    n = B * T * C
    P = lambda t: t.data_ptr()  # noqa: E731

    def fused_fwd():
        _lib.check(lib.wkv4_forward_gated_checkpointed(P(k), P(v), P(td), P(tf), P(r), P(out),
                                                       P(ck), fwp, fws_bytes, B, T, C, code, sp),
                   "gated forward")

    def fused_bwd():
        _lib.check(lib.wkv4_backward_gated_checkpointed(
            P(dy), P(td), P(tf), P(k), P(v), P(r), P(ck), P(gk), P(gv), P(gr), P(gtd), P(gtf),
            P(ws), bws_bytes, B, T, C, code, sp), "gated backward")

    def plain_fwd():
        _lib.check(lib.wkv4_forward_checkpointed(P(k), P(v), P(td), P(tf), P(y), P(ck), fwp,
                                                 fws_bytes, B, T, C, code, sp), "forward")
        _lib.check(lib.sigmoid_gate_forward(P(r), P(y), P(out), n, code, sp), "gate forward")

    def plain_bwd():
        _lib.check(lib.sigmoid_gate_backward(P(dy), P(r), P(y), P(gr), P(gy), n, code, sp),
                   "gate backward")
        _lib.check(lib.wkv4_backward_checkpointed(P(gy), P(td), P(tf), P(k), P(v), P(ck), P(gk),
                                                  P(gv), P(gtd), P(gtf), P(ws), bws_bytes,
                                                  B, T, C, code, sp), "backward")

    variants = {"fused": (fused_fwd, fused_bwd), "unfused": (plain_fwd, plain_bwd)}

    def region(fwd, bwd) -> float:
        for _ in range(args.warmup):
            fwd()
            bwd()
        torch.cuda.synchronize()
        settle_gc()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            fwd()
            bwd()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / args.steps

    res = {}
    for name, (fwd, bwd) in variants.items():
        res[name] = region(fwd, bwd)
    # the same again in the opposite order (box drift shows as a difference)
    for name, (fwd, bwd) in reversed(list(variants.items())):
        res[name] = min(res[name], region(fwd, bwd))
    uses = "fused" if GATED_TIME_MIX else "unfused"
    step_s = res[uses]
    # Algorithmic bytes per element: fused fwd k, v, r read, out written (8);
    # fused bwd k, v, r, dy read, dk, dv, dr written (14).  The unfused pair
    # also writes and reads the WKV output y and its gradient (12 + 20).
    fused_bytes, unfused_bytes = 22 * n, 32 * n
    return {
        "metric": "WKV fwd+bwd with the receptance gate sigmoid(r)*wkv, tokens/sec, "
                  "B=64 T=1024 C=512 bf16",
        "value": B * T / step_s, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": step_s * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "wkv4_gated_fwd_bwd", "B": B, "T": T, "C": C,
                   "io_dtype": "bfloat16", "model_uses": uses},
        "fused_ms_per_step": res["fused"] * 1e3,
        "unfused_ms_per_step": res["unfused"] * 1e3,
        "fused_hbm_gbps_algorithmic": fused_bytes / res["fused"] / 1e9,
        "unfused_hbm_gbps_algorithmic": unfused_bytes / res["unfused"] / 1e9,
        "roofline": {"bound": "hbm", "achieved": (fused_bytes if uses == "fused" else
                                                  unfused_bytes) / step_s / 1e9,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": (fused_bytes if uses == "fused" else unfused_bytes) / step_s / 1e9
                     / HBM_PEAK_GBS, "traffic": None,
                     "kernel": f"{uses} pair, whole step (region time)"},
    }


def bench_timemix(args) -> dict:
    """Fused token-shift mix of the time-mix block (three mixing vectors,
    fp32 input, bf16 outputs) forward + backward through the C ABI on
    preallocated buffers: B=64, T=1024, C=512."""
    import spikegpt_myelin_amd  # noqa: F401
    from spikegpt_myelin_amd import _lib
    from oracle import timemix as TM

    B, T, C, n = 64, 1024, 512, 3
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(B, T, C, generator=g).to(dev)
    mix = torch.rand(n, C, generator=g).to(dev)
    outs = [torch.empty(B, T, C, dtype=torch.bfloat16, device=dev) for _ in range(n)]
    grads = [torch.randn(B, T, C, generator=g).to(torch.bfloat16).to(dev) for _ in range(n)]
    gx = torch.empty_like(x)
    gmix = torch.empty(n, C, dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws = torch.empty(int(lib.token_shift_mix_workspace_bytes(n, B, T, C)), dtype=torch.uint8,
                     device=dev)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    f32, bf16 = _lib.dtype_code(torch.float32), _lib.dtype_code(torch.bfloat16)
    xp, mp = x.data_ptr(), mix.data_ptr()
    op = [o.data_ptr() for o in outs]
    gp = [q.data_ptr() for q in grads]

    def fwd():
        _lib.check(lib.token_shift_mix_forward(xp, f32, mp, n, *op, bf16, B, T, C, sp), "mix fwd")

    def bwd():
        _lib.check(lib.token_shift_mix_backward(xp, f32, mp, n, *gp, bf16, gx.data_ptr(),
                                                gmix.data_ptr(), ws.data_ptr(), ws.numel(),
                                                B, T, C, sp), "mix bwd")

    pool = EventPool(4 * args.steps, stream)
    for _ in range(args.warmup):
        fwd()
        bwd()
    torch.cuda.synchronize()
    evs, fevs = [], []
    settle_gc()
    t0 = time.perf_counter()
    for i in range(args.steps):
        if i % args.event_every == event_offset(args):
            s_ev, e_ev = pool.take(), pool.take()
            _lib.arm_events(s_ev, e_ev)
            fwd()
            fevs.append((s_ev, e_ev))
            s_ev, e_ev = pool.take(), pool.take()
            _lib.arm_events(s_ev, e_ev)
            bwd()
            evs.append((s_ev, e_ev))
        else:
            fwd()
            bwd()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    bwd_t = statistics.mean(s.elapsed_time(e) * 1e-3 for s, e in evs)
    fwd_t = statistics.mean(s.elapsed_time(e) * 1e-3 for s, e in fevs)
    step_s = elapsed / args.steps
    ne = B * T * C
    fwd_bytes, bwd_bytes = (4 + 2 * n) * ne, (4 + 2 * n + 4) * ne
    achieved = bwd_bytes / bwd_t / 1e9
    out = {
        "metric": "fused token-shift mix (3 vectors) fwd+bwd tokens/sec, B=64 T=1024 C=512 "
                  "fp32 in / bf16 out",
        "value": B * T / step_s, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": step_s * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "token_shift_mix_fwd_bwd", "B": B, "T": T, "C": C, "n": n},
        "hbm_gbps_algorithmic": (fwd_bytes + bwd_bytes) / step_s / 1e9,
        "fwd_launch_us": fwd_t * 1e6, "bwd_launch_us": bwd_t * 1e6,
        "fwd_gbps_algorithmic": fwd_bytes / fwd_t / 1e9,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "kernel": "shift_mix_bwd_kernel + column_sum_kernel",
                     "algorithmic_bytes_per_launch": bwd_bytes, "avg_launch_us": bwd_t * 1e6},
    }
    if not args.no_cpu_baseline:
        torch.set_num_threads(os.cpu_count() or 1)
        bs = min(B, args.cpu_sample_batch)
        xc = x[:bs].cpu().requires_grad_(True)
        mc = mix.cpu().requires_grad_(True)
        gc = [q[:bs].float().cpu() for q in grads]
        times = []
        for _ in range(3):
            t1 = time.perf_counter()
            torch.autograd.grad(TM.shift_mix(xc, mc, torch.bfloat16), [xc, mc], gc)
            times.append(time.perf_counter() - t1)
        med = statistics.median(times[1:])
        out["cpu_baseline"] = {
            "value": bs * T / med, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"B={bs} of {B}, T={T}, C={C}, eager token shift + 3 mixes + bf16 cast "
                       f"(language.py:344-353) forward+autograd backward, median of 2 after 1 "
                       f"warmup; host {_cpu_model()}"),
        }
    return out


# Training-step models: (B, T, layers, embedding, vocabulary).  "41m": the
# 41M SpikeGPT (12 x 512, byte vocabulary); "216m": the reference's gpt2-216m
# preset (src/spikegpt/language.py:297-298: 18 layers x 768, context 1024)
# with the GPT-2 BPE vocabulary size 50277, B=16.
E2E_MODELS = {"41m": (64, 1024, 12, 512, 256), "216m": (16, 1024, 18, 768, 50277)}


def bench_e2e(steps: int, warmup: int, model_name: str = "41m") -> dict:
    """A SpikeGPT training step: random init, synthetic tokens, bf16 autocast,
    fused AdamW with gradient clipping -- the recipe of the reference's
    trainer (examples/train_tiny_spikegpt.py:646-655, 797, 866-880).  WKV,
    LIF, token shift, layer norm + mix and the gates run in the HIP kernels;
    GEMMs and the loss are PyTorch-ROCm (hipBLASLt)."""
    from spikegpt_myelin_amd.model import SpikeGPTConfig, SpikeLanguageModel

    B, T, layers, embd, vocab = E2E_MODELS[model_name]
    dev = torch.device("cuda", 0)
    torch.manual_seed(0)
    cfg = SpikeGPTConfig(vocab_size=vocab, context_length=T, n_layer=layers, n_embd=embd,
                         dropout=0.0)
    model = SpikeLanguageModel(cfg).to(dev)
    n_params = sum(p.numel() for p in model.parameters())
    opt = torch.optim.AdamW(model.parameters(), lr=3e-3, weight_decay=0.01, fused=True)
    g = torch.Generator().manual_seed(0)
    ids = torch.randint(0, vocab, (B, T + 1), generator=g).to(dev)
    x, y = ids[:, :-1].contiguous(), ids[:, 1:].contiguous()

    def step():
        opt.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss, _ = model(x, y)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        opt.step()
        return loss

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    settle_gc()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    return {"tokens_per_s": B * T / dt, "ms_per_step": dt * 1e3, "steps": steps,
            "warmup": warmup, "loss_last": float(loss), "params": n_params,
            "config": {"model": f"spikegpt-{model_name}", "n_layer": layers, "n_embd": embd,
                       "vocab": vocab, "B": B, "T": T, "dtype": "bf16 autocast",
                       "optimizer": "AdamW fused, clip 1.0", "data": "synthetic tokens"}}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--event-every", type=int, default=10,
                    help="time the dominant launch with HIP events on every N-th timed step")
    ap.add_argument("--workload", default="wkv4", choices=[*WORKLOADS, "decode", "block_decode", "wkv7", "lif",
                             "timemix", "gated", "e2e41m", "e2e216m"])
    ap.add_argument("--cpu-sample-batch", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--e2e-steps", type=int, default=20,
                    help="timed steps of the 41M SpikeGPT training step reported with the "
                         "default workload (0 skips it)")
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="first run one device copy of this many MiB (a kernel of known traffic "
                         "for scaling PMC byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the WKV recurrence is benchmarked on a single MI355X "
              "(per-GPU throughput at the per-GPU batch); multi-GPU runs are not part of it.",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        return 2
    sys.path.insert(0, str(ROOT))
    if args.calibration_copy_mib:
        src = torch.ones(args.calibration_copy_mib << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.workload == "decode":
        out = bench_decode(args)
    elif args.workload == "block_decode":
        out = bench_block_decode(args)
    elif args.workload == "wkv7":
        out = bench_wkv7(args)
    elif args.workload == "lif":
        out = bench_lif(args)
    elif args.workload == "timemix":
        out = bench_timemix(args)
    elif args.workload == "gated":
        out = bench_gated(args)
    elif args.workload in ("e2e41m", "e2e216m"):
        out = bench_e2e(args.steps, args.warmup, args.workload[3:])
    else:
        out = bench_wkv4(args, WORKLOADS[args.workload])
        if args.workload == "wkv4" and args.e2e_steps > 0:
            out["e2e_train_step"] = bench_e2e(args.e2e_steps, 5)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
