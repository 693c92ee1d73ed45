"""Benchmark of the split-manifold LUT path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--instances N]

Workload: LUT-GEMV 2560 -> 6912 (MLP gate/up),
batch 1, fp32 activations, d = 16 / 256 centroids, 0.38 % CSR outliers.  A
step is one call of the fused LUT-GEMV kernel on one of N distinct weight
instances (round robin, 262 MB at N = 160, above the 256 MB Infinity Cache).

HBM residency: before every timed pass a 512 MiB buffer is read (a sum, no
writes), which evicts the Infinity Cache and the L2s without leaving dirty
lines, so the first N calls of a pass read their codes from HBM whatever K
is; longer passes cycle through a working set above 256 MB.

Printed: one JSON line (kept under 8 KB).  ``value`` is microseconds per call
(lower is better), measured with HIP events on the launch stream over the K
timed back-to-back steps, enqueued behind a bounded spin kernel (the gate) so
the events time the GPU running them, not the host issuing them.
``roofline`` relates the algorithmic code bytes of one launch to the
kernel's own average duration, measured live with the library's start/stop
events (hipExtLaunchKernelGGL: the kernel's begin and end on the launch
stream) over max(K, 200) launches that also run back to back behind a gate
(``gate_held``: the host had enqueued every launch before the gate ended);
for a call that launches one kernel the call period bounds it too, and the
smaller bound is used (kernel_us).
``traffic`` is the HBM bytes per launch from the rocprofv3
FETCH_SIZE / WRITE_SIZE summaries committed under profiles/ (lines
``traffic_bytes_per_launch[<leg>]: <bytes>``).  ``cpu_baseline`` times the
reference's own C++ engine (compiled from its sources into oracle/_ref when
present, else the repo's C restatement) on the host, one thread.

Legs beside the headline (``legs``; each with its call time, its dominant
kernel's roofline and traffic, and a CPU figure where the reference has one):
the 2560 -> 2560 linear, bf16 at batch 1 and the batched linear
(configs[1]), the grouped launch (the sustained form), the MoE layer per
call and as a 16-layer graph, the KV decode and append
(configs[3]), the streamed attention over int8 pages, the 4B-shaped decoder
(configs[4]) and a measured device-to-device copy rate.

Profiling switches (not used by the driver): ``--skip-headline`` runs only
the legs named by ``--extra``; ``--gate-us`` sets the gate's hold per
enqueued call (raise it under a profiler, whose launches cost more host time).
"""
import argparse
import ctypes
import glob
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
M_GU, K_GU = 6912, 2560
CAL_COPY_BYTES = 64 << 20
FLUSH_BYTES = 512 << 20
MIN_KERNEL_LAUNCHES = 200
PROFILES = os.path.join(ROOT, "profiles")
VP = ctypes.c_void_p
ALL_LEGS = ("copy,linear2560,bf16,batched,sustained,moe,moe_sustained,kv,kv_append,attn,"
            "decoder")


def profile_traffic():
    """{leg key: HBM bytes per launch} from every committed rocprofv3 PMC
    summary under profiles/ (lines ``traffic_bytes_per_launch[key]: N``)."""
    out = {}
    for path in sorted(glob.glob(os.path.join(PROFILES, "*.md"))):
        try:
            with open(path) as f:
                for key, val in re.findall(r"traffic_bytes_per_launch\[([\w.-]+)\]:\s*(\d+)",
                                           f.read()):
                    out[key] = int(val)
        except OSError:
            pass
    return out


TRAFFIC = profile_traffic()


def host_info():
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            m = re.search(r"model name\s*:\s*(.+)", f.read())
            model = m.group(1).strip() if m else None
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return {"cpu_model": model, "logical_cpus": os.cpu_count(), "usable_cpus": usable}


def cpu_threads():
    """Threads for the multi-threaded CPU variants: the host share of one GPU
    on the box (16), at most what this process may use."""
    return max(1, min(16, host_info()["usable_cpus"] or 1))


def timed_cpu(call, seconds, max_calls, warm=3):
    """Mean seconds per call of ``call`` over at most ``seconds`` / ``max_calls``
    after ``warm`` untimed calls (ojasx_run.cpp's steady-clock method)."""
    for _ in range(warm):
        call()
    n, t0 = 0, time.perf_counter()
    while True:
        call()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= max_calls:
            return el / n, n


def short(name):
    """Kernel name as recorded by the library, compacted: "XS_" and the spaces
    dropped from a long template list, the list dropped if still long (the
    library records a template launch's parameter names there, not values)."""
    if len(name) <= 26:
        return name
    c = name.replace("XS_", "").replace(", ", ",")
    return c if len(c) <= 30 else name.split("<")[0]


class Bench:
    """Device, stream, library, the cache flush and the gate shared by every leg."""

    def __init__(self, torch, pkg, gate_us):
        self.torch = torch
        self.pkg = pkg
        self.L = pkg.lib()
        self.dev = torch.device("cuda:0")
        self.stream = torch.cuda.current_stream()
        self.sp = VP(self.stream.cuda_stream)
        self.fbuf = torch.zeros(FLUSH_BYTES // 4, device=self.dev)
        self.gate_us = gate_us

    def flush(self):
        """Read 512 MiB (a sum): evicts the Infinity Cache and every L2 without
        leaving dirty lines, whose write-back would otherwise land in the timed
        calls (0.3-0.4 us per call over a 20-call headline pass)."""
        self.fbuf.sum()
        self.torch.cuda.synchronize()

    def gate(self, n, per_call_us):
        """Hold the stream with a bounded spin kernel (per_call_us for each of
        the n calls to come, at least 50 ms, at most 0.2 s) while the host
        enqueues the timed calls.  Returns an event recorded behind it: still
        pending once the calls are enqueued means the gate held."""
        torch = self.torch
        torch.cuda._sleep(int(min(max(n * per_call_us, 50000), 200000) * 2400))
        ev = torch.cuda.Event()
        ev.record(self.stream)
        return ev

    def events_us(self, fn, n, gate=True):
        """Average us per call of fn(i), i < n, from HIP events on the launch
        stream, after a flush, the calls enqueued behind a gate.  Returns
        (us, gate held)."""
        torch = self.torch
        self.flush()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        g = self.gate(n, self.gate_us) if gate else None
        e0.record(self.stream)
        for i in range(n):
            fn(i)
        e1.record(self.stream)
        held = (not g.query()) if g is not None else None
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / n, held

    def kernels(self, fn, n, gate=True):
        """({kernel: {"calls", "avg_us"}}, gate held) of fn(i) over
        max(n, 200) calls from the library's start/stop events, after a flush,
        enqueued behind a gate so the kernels run back to back as in the
        events pass.  A first untimed pass sizes the library's event pool."""
        n = max(n, MIN_KERNEL_LAUNCHES)
        lib = self.pkg._lib
        lib.kernel_timing_enable(True)
        try:
            for i in range(n):
                fn(i)
            lib.kernel_timing_report()
            self.flush()
            lib.kernel_timing_enable(True)
            g = self.gate(n, self.gate_us * 6) if gate else None
            for i in range(n):
                fn(i)
            held = (not g.query()) if g is not None else None
            rep = lib.kernel_timing_report()
        finally:
            lib.kernel_timing_enable(False)
        rep.pop("_dropped", None)
        return rep, held


def frac(nbytes, us):
    return round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 5)


def roofline(code_bytes, all_bytes, kernel_us, kernel, calls, traffic=None):
    """The contract's roofline object for the headline kernel."""
    ach = code_bytes / (kernel_us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 5), "traffic": traffic, "kernel": short(kernel),
            "kernel_avg_us": round(kernel_us, 4), "kernel_launches_timed": calls,
            "algorithmic_bytes_per_launch": int(code_bytes),
            "all_compulsory_bytes_per_launch": int(all_bytes),
            "frac_all_bytes": frac(all_bytes, kernel_us)}


def kernel_us(kern, name, us):
    """(kernel duration, library-event average) in us.  The duration is the
    event average, or, when each call launches this one kernel and nothing
    else, the call period if that is smaller: those calls run back to back,
    so a kernel lasts at most one period, while the events' own overhead
    (about 0.2 us on long kernels, up to 1.2 us on 3 us ones) can lift their
    average above it.  Both are upper bounds of the kernel's duration."""
    ev = kern[name]["avg_us"]
    single = len(kern) == 1
    return (min(ev, us) if single else ev), ev


def leg(us, kern, name, code_bytes, all_bytes, key, held=None):
    """Compact record of one leg: call period, the dominant kernel's duration
    (``kus``, see kernel_us; ``kus_events`` when the event average is larger;
    ``n`` launches timed), its fractions of 8 TB/s on code bytes and on all
    compulsory bytes per launch, and its measured traffic per launch."""
    kus, ev = kernel_us(kern, name, us)
    out = {"us": round(us, 3), "kernel": short(name), "kus": round(kus, 3),
           "n": kern[name]["calls"], "code_B": int(code_bytes), "frac": frac(code_bytes, kus),
           "frac_all": frac(all_bytes, kus), "traffic": TRAFFIC.get(key)}
    if ev > kus:
        out["kus_events"] = round(ev, 3)
    if held is False:
        out["gate_held"] = False
    return out


def sizes(args, default):
    """The sizes a leg runs: its defaults, or --sizes (profiling runs)."""
    return tuple(int(v) for v in args.sizes.split(",")) if args.sizes else default


def dominant(kern):
    return max(kern, key=lambda k: kern[k]["calls"] * kern[k]["avg_us"])


def per_call_us(kern, calls):
    return {short(k): round(v["avg_us"] * v["calls"] / calls, 3) for k, v in kern.items()}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--instances", type=int, default=160)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip every extra figure (headline only)")
    ap.add_argument("--extra", default=ALL_LEGS, help="comma-separated legs to run")
    ap.add_argument("--skip-headline", action="store_true",
                    help="profiling runs only: run just the legs named by --extra")
    ap.add_argument("--gate-us", type=float, default=15.0,
                    help="gate hold per enqueued call, us (raise it under a profiler)")
    ap.add_argument("--sizes", default=None,
                    help="profiling runs only: the batch / token counts of the batched, MoE, "
                         "KV and append legs to run (comma-separated), instead of their defaults")
    return ap.parse_args()


# --- linear legs ------------------------------------------------------------------

def make_instances(b, M, K, n, seed, csr=True):
    """n LUT-GEMV handles M x K: one seeded codebook, scales, CSR (unless csr
    is False) and x, codes drawn per instance.  Returns (handles, base inputs,
    device bytes per handle)."""
    L = b.L
    base = b.pkg.synthetic.linear(M, K, B=64, seed=seed)
    r = np.random.default_rng(seed + 1)
    p = lambda a: a.ctypes.data_as(VP)
    rp, cl, vl = base["csr"]
    hs, wbytes = [], 0
    for i in range(n):
        codes = base["codes"] if i == 0 else r.integers(0, 256, size=base["codes"].shape,
                                                        dtype=np.uint8)
        h = L.ojasx_create_linear(K, M, 16, 256, p(base["codebook"]), p(codes),
                                  p(base["scales"]), None)
        assert h, L.ojasx_get_last_error()
        if csr:
            assert L.ojasx_set_linear_outliers(h, vl.size, p(rp), p(cl), p(vl)) == 0
        hs.append(h)
        wbytes = L.ojasx_linear_device_weight_bytes(h)
    base["nnz"] = vl.size if csr else 0
    return hs, base, wbytes


def cpu_linear(base, B, seconds, y_gpu=None, threads=(1,)):
    """Reference C++ engine (or the C restatement) on the host for one call of
    B tokens: us per call per thread count; its output on instance 0 is the
    parity check of the GPU result (max |GPU - CPU| / max |CPU|)."""
    from oracle import ref, cpu
    x = base["x"][:B]
    if ref.available():
        R = ref.RefLinear(base["codebook"], base["codes"], base["scales"], None, base["csr"])
        mk = lambda nt: (lambda: R.forward(x, nt))
        kind = "reference"
    else:
        mk = lambda nt: (lambda: cpu.linear_forward(x, base["codebook"], base["codes"],
                                                    base["scales"], None, *base["csr"]))
        kind = "port"
        threads = (1,)
    out = {"kind": kind, "batch": B}
    if y_gpu is not None:
        y_cpu = np.asarray(mk(1)(), np.float64).reshape(-1)
        out["rel_err"] = float("%.3g" % (np.abs(np.asarray(y_gpu, np.float64).reshape(-1) - y_cpu)
                                         .max() / np.abs(y_cpu).max()))
    for nt in threads:
        s, n = timed_cpu(mk(nt), seconds, 1000)
        out[f"us_{nt}t"] = round(s * 1e6, 1)
        out[f"calls_{nt}t"] = n
    return out


def linear_leg(b, hs, base, wbytes, M, K, B, dt, steps, warmup, key):
    """us per call (events) and the kernel roofline of ``B``-token calls over
    the instances in round robin (flushed before each pass)."""
    torch, L = b.torch, b.L
    n = len(hs)
    x = torch.from_numpy(base["x"][:B]).to(b.dev)
    if dt:
        x = x.to(torch.bfloat16)
    y = torch.empty(B, M, device=b.dev, dtype=x.dtype)
    xp, yp = VP(x.data_ptr()), VP(y.data_ptr())
    call = lambda i: L.ojasx_linear_forward_device(hs[i % n], xp, yp, B, dt, b.sp)
    assert call(0) == 0, L.ojasx_get_last_error()
    for i in range(max(warmup, n)):   # every instance once: workspaces sized outside the timing
        call(i)
    torch.cuda.synchronize()
    us, held = b.events_us(call, steps)
    kern, kheld = b.kernels(call, steps)
    name = dominant(kern)
    code_bytes = M * (K // 16)
    all_bytes = wbytes + B * K * x.element_size() + B * M * x.element_size()
    if B >= 9:   # the batched kernels read the 32-bit outlier columns
        all_bytes += 2 * base["nnz"]
    out = leg(us, kern, name, code_bytes, all_bytes, key, held and kheld)
    out["TFLOPs"] = round(2.0 * M * K * B / (out["kus"] * 1e-6) / 1e12, 2)
    assert L.ojasx_linear_forward_device(hs[0], xp, yp, B, dt, b.sp) == 0
    torch.cuda.synchronize()
    return out, y.float().cpu().numpy()


def host_pointer_call(b, handles, base, n=200):
    """The reference's own entry point, ojasx_linear_forward (host x and y,
    synchronous: copy in, kernel, copy out), on the headline shape: the
    PCIe-inclusive rate a host-pointer caller sees.  Never the headline value."""
    L = b.L
    x = np.ascontiguousarray(base["x"][:1], np.float32)
    y = np.empty((1, M_GU), np.float32)
    px, py = x.ctypes.data_as(VP), y.ctypes.data_as(VP)
    for i in range(10):
        assert L.ojasx_linear_forward(handles[i % len(handles)], px, py, 1, 1) == 0
    t0 = time.perf_counter()
    for i in range(n):
        L.ojasx_linear_forward(handles[i % len(handles)], px, py, 1, 1)
    us = (time.perf_counter() - t0) / n * 1e6
    return {"us": round(us, 2), "calls": n,
            "code_GBs": round(M_GU * (K_GU // 16) / (us * 1e-6) / 1e9, 1)}


def bench_linear2560(b, args):
    """LUT linear 2560 -> 2560, batch 1, fp32, 0.38 %
    CSR, over 400 instances (268 MB), with the reference engine's CPU time."""
    M = K = 2560
    hs, base, wbytes = make_instances(b, M, K, 400, 2040)
    n = max(MIN_KERNEL_LAUNCHES, min(args.steps, 400))
    try:
        res, y0 = linear_leg(b, hs, base, wbytes, M, K, 1, 0, n, args.warmup, "linear2560")
        if not args.no_cpu:
            c = cpu_linear(base, 1, min(2.0, args.cpu_seconds), y0, threads=(1, cpu_threads()))
            res["cpu"] = {"us": c["us_1t"], "cores": 1, "kind": c["kind"], "rel_err": c["rel_err"],
                          f"us_{cpu_threads()}t": c.get(f"us_{cpu_threads()}t")}
    finally:
        for h in hs:
            b.L.ojasx_destroy_linear(h)
    return res


def bench_nocsr(b, args):
    """Profiling leg (only with --extra nocsr): the headline shape with no
    outliers, for the traffic attribution of the CSR stream."""
    hs, base, wbytes = make_instances(b, M_GU, K_GU, args.instances, 2026, csr=False)
    try:
        res, _ = linear_leg(b, hs, base, wbytes, M_GU, K_GU, 1, 0,
                            max(MIN_KERNEL_LAUNCHES, args.steps), args.warmup, "nocsr_b1")
    finally:
        for h in hs:
            b.L.ojasx_destroy_linear(h)
    return res


def bench_sustained(b, handles, base, wbytes):
    """The same LUT-GEMV on all N weight instances in one grouped launch
    (ojasx_linear_forward_grouped_device): the sustained rate over a working
    set above the Infinity Cache.  Each launch is a whole pass over the 262 MB
    of instances, so the count only sets how steady the average is: 200
    launches whatever --steps is."""
    torch, L = b.torch, b.L
    n = len(handles)
    x = torch.from_numpy(base["x"][:1]).to(b.dev)
    ys = torch.empty(n, M_GU, device=b.dev)
    H = (VP * n)(*handles)
    X = (VP * n)(*([x.data_ptr()] * n))
    Y = (VP * n)(*[ys[i].data_ptr() for i in range(n)])
    call = lambda i: L.ojasx_linear_forward_grouped_device(H, n, X, Y, b.sp)
    for _ in range(3):
        assert call(0) == 0, L.ojasx_get_last_error()
    torch.cuda.synchronize()
    reps = MIN_KERNEL_LAUNCHES
    us, held = b.events_us(call, reps)
    kern, kheld = b.kernels(call, reps)
    kname = dominant(kern)
    code_bytes = n * M_GU * (K_GU // 16)
    all_bytes = n * (wbytes + K_GU * 4 + M_GU * 4)
    out = leg(us, kern, kname, code_bytes, all_bytes, "sustained" if n == 160 else None,
              held and kheld)
    out.update({"instances": n, "us_per_linear": round(out["kus"] / n, 4)})
    return out


def bench_batched(b, handles, base, wbytes, args):
    """LUT-GEMV 2560->6912 at batch 8, 16, 32 and 64,
    fp32 and bf16 activations, over the headline's instances (flushed before
    each pass).  From 17 tokens the call runs as x . W^T on bf16 MFMA over
    exact bf16 pieces (lut_mm32_kernel), from 9 on fp32 MFMA (lut_mm_kernel),
    below that the in-place LUT kernel (lut_dec_kernel).
    CPU: the reference engine at 8 and 64 tokens (it loops tokens)."""
    res = {}
    n = max(MIN_KERNEL_LAUNCHES, min(args.steps, 400))
    y8 = {}
    for dt, tag in ((0, "fp32"), (1, "bf16")):
        for B in sizes(args, (8, 16, 32, 64)):
            r, y0 = linear_leg(b, handles, base, wbytes, M_GU, K_GU, B, dt, n,
                               min(args.warmup, 20), f"{tag}_B{B}")
            res[f"{tag}_B{B}"] = r
            if dt == 0:
                y8[B] = y0
    if not args.no_cpu:
        for B in (B for B in (8, 64) if B in y8):
            c = cpu_linear(base, B, min(1.5, args.cpu_seconds), y8[B], threads=(1,))
            res[f"fp32_B{B}"]["cpu"] = {"us": c["us_1t"], "cores": 1, "kind": c["kind"],
                                        "rel_err": c["rel_err"]}
    return res


# --- MoE ----------------------------------------------------------------------------

E_MOE, H_MOE, I_MOE, K_MOE = 512, 2048, 768, 10
GU_BYTES = 2 * I_MOE * (H_MOE // 16)      # gate/up code bytes per expert
DN_BYTES = H_MOE * (I_MOE // 16)          # down code bytes per expert
SC_BYTES = (2 * I_MOE + H_MOE) * 4        # scales per expert


def moe_banks(b):
    L = b.L
    gen = b.pkg.synthetic
    p = lambda a: a.ctypes.data_as(VP)
    banks = []
    for seed in (11, 12):
        m = gen.moe(E=E_MOE, H=H_MOE, I=I_MOE, T=256, seed=seed)
        h = L.ojasx_create_moe(E_MOE, H_MOE, I_MOE, K_MOE, 16, p(m["cb_in"]), p(m["cb_down"]),
                               p(m["gu_codes"]), p(m["gu_scales"]), p(m["dn_codes"]),
                               p(m["dn_scales"]))
        assert h, L.ojasx_get_last_error()
        banks.append((h, m))
    return banks


def moe_route(b, T, n, seed):
    torch, L = b.torch, b.L
    r = np.random.default_rng(seed)
    logits = torch.from_numpy(r.normal(size=(n, T, E_MOE)).astype(np.float32)).to(b.dev)
    idx = torch.empty(n, T, K_MOE, dtype=torch.int32, device=b.dev)
    w = torch.empty(n, T, K_MOE, dtype=torch.float32, device=b.dev)
    for i in range(n):
        assert L.ojasx_moe_route_device(VP(logits[i].data_ptr()), T, E_MOE, K_MOE, 0,
                                        VP(idx[i].data_ptr()), VP(w[i].data_ptr()), b.sp) == 0
    torch.cuda.synchronize()
    distinct = np.array([len(np.unique(a)) for a in idx.cpu().numpy().reshape(n, -1)])
    return idx, w, distinct


def moe_dominant_bytes(name, experts):
    """Algorithmic code bytes per launch of an MoE kernel: the gate/up or down
    codes of the distinct routed experts (the kernels reading codes)."""
    if "SWIGLU" in name or "down" in name:
        return experts * DN_BYTES
    return experts * GU_BYTES


def bench_moe(b, args):
    """512-expert top-10 MoE layer (H 2048, I 768), T = 1 and 16 tokens.  Two
    expert banks (2 x 151 MB, above the 256 MB Infinity Cache) alternate and
    every step has its own routing (routed on the device); code bytes count
    the distinct experts a call reads.  CPU: the reference engine, whose API
    is one token per call (16 calls for T = 16)."""
    from oracle import ref
    torch, L = b.torch, b.L
    banks = moe_banks(b)
    res = {}
    nsteps = max(MIN_KERNEL_LAUNCHES, min(args.steps, 400))
    try:
        for T in sizes(args, (1, 16)):
            idx, w, distinct = moe_route(b, T, nsteps, T)
            x = torch.from_numpy(banks[0][1]["x"][:T]).to(b.dev)
            y = torch.empty(T, H_MOE, device=b.dev)
            fwd = lambda i: L.ojasx_moe_forward_device(banks[i % 2][0], VP(x.data_ptr()),
                                                       VP(idx[i].data_ptr()), VP(w[i].data_ptr()),
                                                       VP(y.data_ptr()), T, K_MOE, 0, b.sp)
            for i in range(min(args.warmup, nsteps)):
                fwd(i)
            torch.cuda.synchronize()
            us, held = b.events_us(fwd, nsteps)
            kern, kheld = b.kernels(fwd, nsteps)
            U = float(distinct.mean())
            name = dominant(kern)
            code = U * (GU_BYTES + DN_BYTES)
            kb = moe_dominant_bytes(name, U)
            r = leg(us, kern, name, kb, kb + U * SC_BYTES / 2, f"moe_T{T}", held and kheld)
            r.update({"experts": U, "code_B_call": int(code), "frac_call": frac(code, us),
                      "kernels_us": per_call_us(kern, kern[name]["calls"])})
            res[f"T{T}"] = r
            if not args.no_cpu and ref.available():
                m = banks[0][1]
                R = ref.RefMoE(m["cb_in"], m["cb_down"], m["gu_codes"], m["gu_scales"],
                               m["dn_codes"], m["dn_scales"])
                ii = idx[0].cpu().numpy()
                ww = w[0].cpu().numpy()
                call = lambda: [R.forward(m["x"][t], ii[t], ww[t]) for t in range(T)]
                s, n = timed_cpu(call, min(2.0, args.cpu_seconds), 100, warm=1)
                r["cpu"] = {"us": round(s * 1e6, 1), "cores": 1, "kind": "reference",
                            "sample": f"{n} calls x {T} token(s)"}
    finally:
        for h, _ in banks:
            L.ojasx_destroy_moe(h)
    return res


def moe_sustained_one(b, banks, T, n_layers=16, replays=5):
    """n_layers MoE layers, each on the next of the two alternating expert
    banks with its own device routing, layer i's output the input of layer
    i + 1, captured as one HIP graph and replayed after a flush: the steady
    state of a deep MoE stack (302 MB of banks per pair of layers).  The
    replay's output is compared with an eager run of the same layers."""
    torch, L = b.torch, b.L
    idx, w, distinct = moe_route(b, T, n_layers, 1000 + T)
    xs = [torch.zeros(T, H_MOE, device=b.dev) for _ in range(n_layers + 1)]
    xs[0].copy_(torch.from_numpy(banks[0][1]["x"][:T]))

    def layers(sp):
        for i in range(n_layers):
            rc = L.ojasx_moe_forward_device(banks[i % 2][0], VP(xs[i].data_ptr()),
                                            VP(idx[i].data_ptr()), VP(w[i].data_ptr()),
                                            VP(xs[i + 1].data_ptr()), T, K_MOE, 0, sp)
            assert rc == 0, L.ojasx_get_last_error()

    layers(b.sp)                                     # eager: sizes every workspace
    torch.cuda.synchronize()
    eager = xs[n_layers].clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s), torch.cuda.graph(g, stream=s):
        layers(VP(s.cuda_stream))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    same = bool(torch.equal(xs[n_layers], eager))
    b.flush()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(b.stream)
    for _ in range(replays):
        g.replay()
    e1.record(b.stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (replays * n_layers)
    # the eager layers' kernels, timed back to back, for the per-kernel split
    kern, held = b.kernels(lambda i: layers(b.sp) if i % n_layers == 0 else None,
                           n_layers * 4, gate=True)
    del g
    U = float(distinct.mean())
    code = U * (GU_BYTES + DN_BYTES)
    name = dominant(kern)
    calls = kern[name]["calls"]
    kb = moe_dominant_bytes(name, U)
    return {"us": round(us, 3), "experts": U, "code_B": int(code), "frac_call": frac(code, us),
            "kernel": short(name), "kus": round(kern[name]["avg_us"], 3), "n": calls,
            "frac": frac(kb, kern[name]["avg_us"]),
            "traffic": TRAFFIC.get(f"moe_sus_T{T}", TRAFFIC.get(f"moe_T{T}")),
            "kernels_us": per_call_us(kern, calls), "graph_equals_eager": same}


def bench_moe_sustained(b, args):
    """16 layers of T = 16, 64 and 256 tokens in one HIP graph (see
    moe_sustained_one)."""
    banks = moe_banks(b)
    try:
        return {f"T{T}": moe_sustained_one(b, banks, T) for T in sizes(args, (16, 64, 256))}
    finally:
        for h, _ in banks:
            b.L.ojasx_destroy_moe(h)


# --- KV decode ----------------------------------------------------------------------

def bench_kv(b, args):
    """Paged code-domain decode, 8 kv / 32 q heads, head_dim 128, page 16, at
    2048 and 32768 tokens.  Every call reads another layer's cache (codes,
    scales and codebooks of its own), over more than 256 MB of caches, after a
    flush.  CPU: the reference engine's ojasx_kv_cache_attention for the 32
    query heads (one call per query head, its kv head j // 4; the reference
    re-reads each kv head's codes for every query head) over the same number
    of tokens appended by its scalar quantiser."""
    from oracle import ref
    torch, L = b.torch, b.L
    res = {}
    Hkv, Hq, hd, P = 8, 32, 128, 16
    g = torch.Generator(device=b.dev).manual_seed(5)
    for T in sizes(args, (2048, 32768)):
        pages = T // P
        per_layer = 2 * pages * Hkv * P * 8 + 2 * pages * Hkv * P * 4 + 2 * Hkv * 256 * 16 * 4
        layers = max(2, -(-(300 << 20) // per_layer))
        kc = torch.randint(0, 256, (layers, pages, Hkv, P, 8), dtype=torch.uint8, device=b.dev,
                           generator=g)
        vc = torch.randint(0, 256, (layers, pages, Hkv, P, 8), dtype=torch.uint8, device=b.dev,
                           generator=g)
        ks = torch.rand(layers, pages, Hkv, P, device=b.dev, generator=g) + 0.5
        vs = torch.rand(layers, pages, Hkv, P, device=b.dev, generator=g) + 0.5
        kcb = torch.randn(layers, Hkv, 256, 16, device=b.dev, generator=g)
        vcb = torch.randn(layers, Hkv, 256, 16, device=b.dev, generator=g)
        bt = torch.randperm(pages, device=b.dev, generator=g).to(torch.int32)
        q = torch.randn(Hq, hd, device=b.dev, generator=g)
        out = torch.empty(Hq, hd, device=b.dev)
        ptr = lambda t, l: VP(t[l].data_ptr())
        call = lambda i: L.ojasx_kv_decode_paged_device(
            VP(q.data_ptr()), ptr(kc, i % layers), ptr(ks, i % layers), ptr(vc, i % layers),
            ptr(vs, i % layers), ptr(kcb, i % layers), ptr(vcb, i % layers), VP(bt.data_ptr()),
            T, P, Hq, Hkv, hd, 16, -1.0, VP(out.data_ptr()), b.sp)
        assert call(0) == 0, L.ojasx_get_last_error()
        for i in range(min(args.warmup, 20)):
            call(i)
        torch.cuda.synchronize()
        n = max(MIN_KERNEL_LAUNCHES, min(args.steps, 400))
        us, held = b.events_us(call, n)
        kern, kheld = b.kernels(call, n)
        code_bytes = 2 * T * Hkv * 8
        all_bytes = code_bytes + 2 * T * Hkv * 4 + 2 * Hkv * 256 * 16 * 4
        name = dominant(kern)
        r = leg(us, kern, name, code_bytes, all_bytes, f"kv_T{T}", held and kheld)
        r.update({"layers_rotated": layers, "frac_all_call": frac(all_bytes, us),
                  "kernels_us": per_call_us(kern, kern[name]["calls"])})
        res[f"T{T}"] = r
        del kc, vc, ks, vs, kcb, vcb
        if not args.no_cpu and ref.available():
            R = ref.RefKV(Hkv, hd, T, 16)
            rg = np.random.default_rng(T)
            kv = rg.normal(size=(T, 2, Hkv, hd)).astype(np.float32)
            for t in range(T):
                for h in range(Hkv):
                    R.append(h, kv[t, 0, h], kv[t, 1, h])
            qh = rg.normal(size=(Hq, hd)).astype(np.float32)
            outh = np.zeros(hd, np.float32)
            pq = [qh[j].ctypes.data_as(VP) for j in range(Hq)]
            po = outh.ctypes.data_as(VP)
            RL = ref.lib()
            call_cpu = lambda: [RL.ojasx_kv_cache_attention(R.h, j // (Hq // Hkv), pq[j], po, -1.0)
                                for j in range(Hq)]
            s, m = timed_cpu(call_cpu, min(2.0, args.cpu_seconds), 1000)
            r["cpu"] = {"us": round(s * 1e6, 1), "cores": 1, "kind": "reference",
                        "sample": f"{m} decodes x 32 q heads"}
            del R
    return res


def bench_attn_pages(b, args, T=32768, page=256, n_caches=4):
    """OnlineSoftmaxBlockAttention.forward_stream over the int8 pages of a
    PagedCompressedKVCache read in place: 32 query / 8 kv heads, head_dim 128,
    one decode query, T tokens in pages of 256, fp64 state.  Calls rotate over
    n_caches caches (more than 256 MB) after a flush; each call is the whole
    Python face (init, update, merge, finalize and the report's max_logsumexp,
    which synchronises, so no gate).  CPU: the fp64 NumPy restatement of
    forward_stream over the same cache's dequantised pages, 1 thread."""
    from oracle import numpy_oracle as no
    torch = b.torch
    lc = b.pkg.long_context
    B, Hq, Hkv, D = 1, 32, 8, 128
    caches = []
    g = torch.Generator(device=b.dev).manual_seed(77)
    for _ in range(n_caches):
        c = lc.PagedCompressedKVCache(page_size=page, max_resident_pages=T // page + 2,
                                      sink_pages=2)
        for t0 in range(0, T, 4096):
            c.append(torch.randn(B, Hkv, 4096, D, device=b.dev, generator=g),
                     torch.randn(B, Hkv, 4096, D, device=b.dev, generator=g))
        caches.append(c)
    attn = lc.OnlineSoftmaxBlockAttention(Hq, Hkv, D, causal=False)
    q = torch.randn(B, Hq, 1, D, device=b.dev, generator=g, dtype=torch.float32)
    call = lambda i: attn.forward_stream(q, caches[i % n_caches])
    for i in range(min(args.warmup, 8)):
        call(i)
    torch.cuda.synchronize()
    n = max(40, min(args.steps, 200))
    us, _ = b.events_us(call, n, gate=False)
    kern, _ = b.kernels(call, n, gate=False)
    code = T * Hkv * 2 * D
    all_bytes = code + T * Hkv * 2 * 2
    tile = [k for k in kern if k.startswith("attn_tile_kernel")][0]
    res = leg(us, kern, tile, code, all_bytes, "attn_tile")
    res.update({"tokens": T, "page": page, "caches_rotated": n_caches,
                "kernels_us": {short(k): round(v["avg_us"], 3) for k, v in kern.items()},
                "fp64_TFLOPs": round(4 * T * Hq * D / (kern[tile]["avg_us"] * 1e-6) / 1e12, 2)})
    if not args.no_cpu:
        from threadpoolctl import threadpool_limits
        c = caches[0]
        pages = [(no.paged_dequantize_int8(qk.cpu().numpy(), sk.cpu().numpy()),
                  no.paged_dequantize_int8(qv.cpu().numpy(), sv.cpu().numpy()))
                 for qk, sk, qv, sv in c._pages]
        qn = q.double().cpu().numpy()
        with threadpool_limits(1):
            s, m = timed_cpu(lambda: no.block_attention_stream(qn, pages, False),
                             min(10.0, args.cpu_seconds), 5, warm=1)
        want = no.block_attention_stream(qn, pages, False)[0]
        got = attn.forward_stream(q.double(), c)[0].cpu().numpy()
        res["cpu"] = {"us": round(s * 1e6, 1), "cores": 1, "kind": "port",
                      "sample": f"{m} calls, NumPy fp64 forward_stream",
                      "rel_err_fp64": float("%.3g" % (np.abs(got - want).max()
                                                      / np.abs(want).max()))}
    return res


def bench_kv_append(b, args, cpu_seconds=2.0):
    """Device KV append (encode + paged write) for 8 kv heads x 128, per call
    of 1 or 16 tokens, with the 256 x 16 codebooks (nearest centroid) and with
    the reference's scalar quantiser; each call writes fresh slots of a
    4096-page pool.  Beside it the reference engine's ojasx_kv_cache_append
    on the host, 8 heads per token."""
    from oracle import ref
    torch, L = b.torch, b.L
    Hkv, hd, D, P, pages = 8, 128, 16, 16, 4096
    r = np.random.default_rng(17)
    kc = torch.zeros(pages, Hkv, P, hd // D, dtype=torch.uint8, device=b.dev)
    vc = torch.zeros_like(kc)
    ks = torch.zeros(pages, Hkv, P, device=b.dev)
    vs = torch.zeros_like(ks)
    cb = torch.from_numpy(r.normal(0, 30, size=(2, Hkv, 256, D)).astype(np.float32)).to(b.dev)
    res = {}
    n = max(MIN_KERNEL_LAUNCHES, min(args.steps, 400))
    for tokens in sizes(args, (1, 16)):
        kv = torch.from_numpy(r.normal(size=(2, n, tokens, Hkv, hd)).astype(np.float32)).to(b.dev)
        slots = torch.arange(n * tokens, dtype=torch.int32, device=b.dev).view(n, tokens)
        for mode in ("codebook", "scalar"):
            cbk = VP(cb[0].data_ptr()) if mode == "codebook" else None
            cbv = VP(cb[1].data_ptr()) if mode == "codebook" else None
            call = lambda i: L.ojasx_kv_encode_append_device(
                VP(kv[0, i].data_ptr()), VP(kv[1, i].data_ptr()), tokens, Hkv, hd, D, cbk, cbv,
                VP(slots[i].data_ptr()), P, pages, VP(kc.data_ptr()), VP(ks.data_ptr()),
                VP(vc.data_ptr()), VP(vs.data_ptr()), b.sp)
            for i in range(min(n, 20)):
                call(i)
            torch.cuda.synchronize()
            us, held = b.events_us(call, n)
            kern, kheld = b.kernels(lambda i: call(i % n), n)
            name = dominant(kern)
            in_bytes = 2 * tokens * Hkv * hd * 4
            out_bytes = 2 * tokens * Hkv * (hd // D + 4)
            res[f"{mode}_{tokens}tok"] = leg(us, kern, name, in_bytes, in_bytes + out_bytes,
                                             f"kv_append_{mode}_{tokens}tok", held and kheld)
    if not args.no_cpu and ref.available():
        R = ref.lib()
        h = R.ojasx_create_kv_cache(Hkv, hd, 1 << 17, D)
        k = r.normal(size=(Hkv, hd)).astype(np.float32)
        p = lambda a: a.ctypes.data_as(VP)
        count, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < cpu_seconds and count < 100000:
            for head in range(Hkv):
                R.ojasx_kv_cache_append(h, head, p(k[head]), p(k[head]))
            count += 1
        res["cpu"] = {"us_per_token": round((time.perf_counter() - t0) / count * 1e6, 2),
                      "cores": 1, "kind": "reference",
                      "sample": f"{count} tokens x {Hkv} heads, scalar quantiser"}
        R.ojasx_destroy_kv_cache(h)
    return res


# --- decoder ------------------------------------------------------------------------

class _CpuLinear:
    """One LUT linear through the C restatement of the reference engine's
    forward (oracle/lut_oracle.c), 1 thread, as ``op @ x``."""

    def __init__(self, w):
        self.w = w

    def __matmul__(self, x):
        from oracle import cpu
        w = self.w
        return cpu.linear_forward(np.asarray(x, np.float32), w["codebook"], w["codes"], None, None,
                                  *w["csr"]).astype(np.float64)


def bench_decoder(b, args, n_tokens=128, context=4096):
    """The 4B-shaped LUT decoder (hidden 2560, 36 layers, 32 q / 8 kv heads,
    MLP 9728, LUT LM head over 151936 tokens): greedy decode of n_tokens at a
    4096-token code KV context, one HIP graph per token and eager launches.
    Seeded random weights and context (synthetic_decoder).  Bytes per token:
    codes + CSR of every linear, the KV codes and scales read, and the
    embedding row.  CPU: one token of the same decoder on the host (the C
    restatement of the reference engine for every linear, 1 thread; NumPy
    norms, RoPE and attention); the reference has no decoder of its own."""
    from oracle import numpy_oracle as no
    decm = b.pkg.decoder
    cfg = decm.DecoderConfig(max_steps=n_tokens, max_context=context + n_tokens)
    keep = not args.no_cpu
    d, weights = decm.synthetic_decoder(cfg, context=context, seed=3, device="cuda:0",
                                        keep_weights=keep)
    res = {"tokens": n_tokens, "context": context}
    runs = {}
    for mode, graph in (("graph", True), ("eager", False)):
        d.reset(context)
        d.generate(1, 4, use_graph=graph)          # warm-up (captures the graph)
        d.reset(context)
        b.flush()
        t0 = time.perf_counter()
        toks = d.generate(1, n_tokens, use_graph=graph)
        el = time.perf_counter() - t0
        runs[mode] = toks
        res[f"ms_per_token_{mode}"] = round(el / n_tokens * 1e3, 4)
    res["tokens_per_s"] = round(1e3 / res["ms_per_token_graph"], 1)
    res["graph_equals_eager"] = bool(np.array_equal(runs["graph"], runs["eager"]))
    d.reset(context)
    b.flush()
    b.pkg._lib.kernel_timing_enable(True)
    try:
        d.generate(1, 8, use_graph=False)
        kern = b.pkg._lib.kernel_timing_report()
    finally:
        b.pkg._lib.kernel_timing_enable(False)
    kern.pop("_dropped", None)
    res["kernels_us_per_token"] = {
        short(k): round(v["avg_us"] * v["calls"] / 8, 1)
        for k, v in sorted(kern.items(), key=lambda kv: -kv[1]["avg_us"] * kv[1]["calls"])}
    res["launches_per_token"] = sum(v["calls"] for v in kern.values()) // 8
    qkv, o, gu, dn = 6144, 2560, 19456, 2560
    shapes = [(qkv, 2560), (o, 4096), (gu, 2560), (dn, 9728)]
    dens = 0.0038
    per_layer_codes = sum(M * K // 16 for M, K in shapes)
    # outliers: 16-bit column + fp32 value per entry, and the row pointers
    per_layer_csr = sum(round(dens * M * K) * 6 + (M + 1) * 4 for M, K in shapes)
    lm_codes = cfg.vocab * 160
    lm_csr = round(dens * cfg.vocab * 2560) * 6 + (cfg.vocab + 1) * 4
    kv_bytes = 36 * 8 * (context + n_tokens // 2) * (2 * 8 + 2 * 4)
    code_bytes = 36 * per_layer_codes + lm_codes
    all_bytes = code_bytes + 36 * per_layer_csr + lm_csr + kv_bytes
    ms = res["ms_per_token_graph"]
    res.update({"code_B_token": code_bytes, "all_B_token": int(all_bytes),
                "frac_code": frac(code_bytes, ms * 1e3), "frac_all": frac(all_bytes, ms * 1e3),
                "traffic_per_token": TRAFFIC.get("decoder_token")})
    if keep:
        emb = weights["embedding"]
        caches = [d.read_kv(l, 0, context + 1) for l in range(cfg.layers)]
        t0 = time.perf_counter()
        no.decoder_step(emb[1], weights, cfg, context, caches, {}, linear=_CpuLinear)
        el = time.perf_counter() - t0
        res["cpu"] = {"ms_per_token": round(el * 1e3, 1), "cores": 1, "kind": "port",
                      "sample": "one token: linears on the C restatement, rest NumPy fp64"}
    d.close()
    return res


def copy_peak(b):
    """Device-to-device copy of 1 GiB (read + write counted): a measured HBM
    rate beside the 8 TB/s spec."""
    torch = b.torch
    n = (1 << 30) // 4
    src = torch.ones(n, device=b.dev)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(b.stream)
    for _ in range(10):
        dst.copy_(src)
    e1.record(b.stream)
    torch.cuda.synchronize()
    s = e0.elapsed_time(e1) * 1e-3 / 10
    del src, dst
    return {"GBs": round((2 << 30) / s / 1e9, 1), "frac": round((2 << 30) / s / 1e9 / HBM_PEAK_GBS, 4)}


def headline(b, args, handles, base, wbytes):
    """The headline: K back-to-back calls of the 2560 -> 6912 B = 1 fp32
    LUT-GEMV over the instances, with the kernel's roofline and the CPU
    baseline."""
    torch, L = b.torch, b.L
    n = len(handles)
    x = torch.from_numpy(base["x"][:1]).to(b.dev)
    y = torch.empty(1, M_GU, device=b.dev)
    xp, yp = VP(x.data_ptr()), VP(y.data_ptr())
    fwd = L.ojasx_linear_forward_device
    call = lambda i: fwd(handles[i % n], xp, yp, 1, 0, b.sp)
    assert call(0) == 0, L.ojasx_get_last_error()
    torch.cuda.synchronize()
    y_bench = y.cpu().numpy()

    for i in range(args.warmup):
        call(i)
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    us_call, held = b.events_us(call, args.steps)
    t_wall = time.perf_counter() - t_wall
    code_bytes = M_GU * (K_GU // 16)
    all_bytes = wbytes + K_GU * 4 + M_GU * 4
    kern, kheld = b.kernels(call, args.steps)
    kname = dominant(kern)
    kus, ev = kernel_us(kern, kname, us_call)
    rf = roofline(code_bytes, all_bytes, kus, kname, kern[kname]["calls"], TRAFFIC.get("headline"))
    if ev > kus:
        rf["kernel_events_us"] = round(ev, 4)
    rf["call_period_frac"] = frac(code_bytes, us_call)
    rf["gate_held"] = bool(held and kheld)

    out = {
        "metric": "LUT-GEMV 2560->6912 us/call (HBM GB/s on code bytes alongside)",
        "value": round(us_call, 4),
        "unit": "us/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_call / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) x, N(0,0.02) codebook, uniform codes, 0.38% CSR)",
        "config": {"workload": "LUT-GEMV 2560->6912 gate/up, B=1, fp32, d=16/256 centroids, "
                               "0.38% CSR outliers", "batch": 1, "in_features": K_GU,
                   "out_features": M_GU, "weight_instances": n,
                   "working_set_MB": round(n * wbytes / 2**20, 1)},
        "roofline": rf,
        "wall_s_timed": round(t_wall, 3),
        "host_pointer_call": host_pointer_call(b, handles, base),
    }
    if not args.no_cpu:
        c = cpu_linear(base, 1, args.cpu_seconds, y_bench, threads=(1,))
        out["cpu_baseline"] = {"value": c["us_1t"], "unit": "us/call", "cores": 1,
                               "kind": c["kind"],
                               "sample": f"{c['calls_1t']} calls of LUT-GEMV 2560->6912 B=1 fp32 "
                                         "with CSR, 1 thread, after 3 warm-up calls",
                               "rel_err": c["rel_err"]}
        if c["kind"] == "reference":
            from oracle import ref
            var = {}
            for tag, path in (("scalar", ref.LIB_SCALAR), ("avx2", ref.LIB_AVX2)):
                if not ref.available(path):
                    continue
                R = ref.RefLinear(base["codebook"], base["codes"], base["scales"], None,
                                  base["csr"], path=path)
                for nt in sorted({1, cpu_threads()}):
                    s, _ = timed_cpu(lambda: R.forward(base["x"][:1], nt),
                                     min(2.0, args.cpu_seconds), 1000)
                    var[f"{tag}_{nt}t"] = round(s * 1e6, 1)
            out["cpu_baseline"]["variants_us"] = var
    out["host"] = host_info()
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the path would shard by output rows / experts / kv heads, see DESIGN.md)",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import __graft_entry__

    pkg = __graft_entry__.load_package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    b = Bench(torch, pkg, args.gate_us)
    L = b.L
    extra = set() if args.no_extra else set(args.extra.split(","))

    # PMC calibration: one device-to-device copy of known size (read and write)
    cal_src = torch.ones(CAL_COPY_BYTES // 4, device=dev)
    cal_dst = torch.empty_like(cal_src)
    cal_dst.copy_(cal_src)
    torch.cuda.synchronize()
    del cal_src, cal_dst

    out = {}
    legs = {}
    handles, base, wbytes = make_instances(b, M_GU, K_GU, args.instances, 2026)
    try:
        if not args.skip_headline:
            out = headline(b, args, handles, base, wbytes)
        if "copy" in extra:
            legs["hbm_copy"] = copy_peak(b)
        if "bf16" in extra:
            legs["bf16_b1"], _ = linear_leg(b, handles, base, wbytes, M_GU, K_GU, 1, 1,
                                            max(MIN_KERNEL_LAUNCHES, args.steps), args.warmup,
                                            "bf16_b1")
        if "sustained" in extra:
            legs["sustained"] = bench_sustained(b, handles, base, wbytes)
        if "batched" in extra:
            legs["batched"] = bench_batched(b, handles, base, wbytes, args)
    finally:
        for h in handles:
            L.ojasx_destroy_linear(h)
    if "linear2560" in extra:
        legs["linear2560_b1"] = bench_linear2560(b, args)
    if "nocsr" in extra:
        legs["nocsr_b1"] = bench_nocsr(b, args)
    if "moe" in extra:
        legs["moe"] = bench_moe(b, args)
    if "moe_sustained" in extra:
        legs["moe_graph16"] = bench_moe_sustained(b, args)
    if "kv" in extra:
        legs["kv_decode"] = bench_kv(b, args)
    if "kv_append" in extra:
        legs["kv_append"] = bench_kv_append(b, args)
    if "attn" in extra:
        legs["attn_stream"] = bench_attn_pages(b, args)
    if "decoder" in extra:
        legs["decoder"] = bench_decoder(b, args)
    out["legs"] = legs
    print(json.dumps(out, separators=(",", ":")))


if __name__ == "__main__":
    main()
