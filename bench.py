#!/usr/bin/env python3
"""Benchmark of the three recurrent operators on one MI355X.

    python bench.py [--steps K] [--warmup W] [--settle-ms S] [--gpus 1]

A step is one SelectiveScanFn call over the Mamba-2.8B-layer workload
(batch 8, d_inner 5120, seqlen 2048, dstate 16, variable B/C, softplus, D,
delta_bias, z present), inputs resident in HBM.  Untimed calls of the same
operator for S ms (clock settle), W untimed steps, then K timed steps
bracketed by torch.cuda.synchronize(); rank 0 prints one JSON
line on stdout (progress goes to stderr).  GatedDeltaNet2Fn (4 x 4096 x 16
heads, dk = dv = 128, with initial state) and Mamba3SisoFn (4 x 4096 x 32
heads, P = 64, N = 128) are timed the same way and reported under "ops".

The settle phase is there because the GPU's power management reacts to a
VALU-heavy load started from idle: the first calls run at ~0.36 ms, the
next ~40 at up to 0.48 ms, and from about call 100 on the selective scan
holds ~0.34 ms.  K steps taken right after W = 3 would time that transient
rather than sustained throughput.

Throughput is tokens/s = batch * seqlen / time; the roofline figures use the
algorithmic bytes of xmetai_onnx_plugins.workloads (unique input bytes the
output depends on + output bytes) over the HIP-event time of the kernel(s).
The CPU baseline is the NumPy fp32 sequential recurrence of oracle/ (the
reference CPU path) on a bounded sample of the same workload, timed on this
host, scaled to the full workload by its (linear) cost.

--mode profile-<op> runs only that operator (for rocprofv3), --mode copy
runs the plain device copy used to calibrate the FETCH_SIZE/WRITE_SIZE
counters.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "xmetai-onnx-plugins_amd")
for _p in (ROOT, PKG_DIR):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "tokens/s per op (GDN-2, sel-scan, Mamba-3) + % HBM roofline, 1 MI355X"
HBM_PEAK_GBPS = 8000.0
# Compute ceilings of one MI355X at 2.4 GHz: 256 CUs x 4 SIMDs x 16 lanes of
# non-packed fp32 VALU (lane-instructions/s), and dense fp32 MFMA.
VALU_LANE_OPS = 256 * 4 * 16 * 2.4e9
MFMA_F32_FLOPS = 157.3e12


def floors_us(name, s, nbytes):
    """Lower bounds on one call's time, in microseconds.

    hbm: algorithmic bytes at 8 TB/s.  valu: the essential per-element
    instruction slots of the sequential recurrence (SS: delta*A, B*delta_u,
    the state and output FMAs, and exp2, which issues at 26.5 lane-ops per CU
    per cycle against 63 for v_fma_f32 on MI355X (independent chains, all
    CUs), i.e. 2.4 slots: 6.4 per state-token;
    GDN-2: 4 per state element per token; Mamba-3: decay, readout, update =
    3), at one slot per lane per cycle; where a chunked form runs it is
    reported as valu_sequential_form.  mfma: the fp32 MFMA flops of the
    16-token chunked forms: GDN-2 (head_k <= 512) 96*K*V + 512*V per
    chunk-head in the recurrence (E'S, R'S, the update, (M T) Y) and
    1536*K + 8192 in the preparation (A', M', T^T Ut', M T), K and V padded
    to 16; Mamba-3 (N <= 256) 32*(80*N + 512) per
    chunk and 32-row block (N padded to 64)."""
    f = {"hbm": nbytes / (HBM_PEAK_GBPS * 1e9) * 1e6}
    if name == "selective_scan":
        f["valu"] = s.batch * s.dim * s.seqlen * s.dstate * 6.4 / VALU_LANE_OPS * 1e6
    elif name == "gated_deltanet2":
        f["valu_sequential_form"] = s.batch * s.seqlen * s.nheads * s.dk * s.dv * 4 / VALU_LANE_OPS * 1e6
        if s.dk <= 512:
            kp, vp = -(-s.dk // 16) * 16, -(-s.dv // 16) * 16
            chunks = s.batch * s.nheads * -(-s.seqlen // 16)
            f["mfma"] = chunks * (96 * kp * vp + 512 * vp + 1536 * kp + 8192) / MFMA_F32_FLOPS * 1e6
    elif name == "mamba3_siso":
        f["valu_sequential_form"] = s.batch * s.seqlen * s.nheads * s.headdim * s.dstate * 3 / VALU_LANE_OPS * 1e6
        if s.dstate <= 256:
            np_ = -(-s.dstate // 64) * 64
            chunks = s.batch * s.nheads * -(-s.headdim // 32) * -(-s.seqlen // 16)
            f["mfma"] = chunks * 32 * (80 * np_ + 512) / MFMA_F32_FLOPS * 1e6
    return {k: round(v, 1) for k, v in f.items()}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------

def make_ops():
    from xmetai_onnx_plugins import workloads as W
    import xmetai_onnx_plugins as xp

    def ss():
        s = W.SS_2P8B
        keys = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
        # z is a dead input of output 0 (never read by the kernel); it is drawn
        # on the device instead of on the host to keep the set-up short.
        host_shape = W.SelectiveScanShape(s.batch, s.dim, s.seqlen, s.dstate, has_z=False)
        return dict(name="selective_scan", workload="selective_scan_b8_d5120_l2048_n16", shape=s,
                    gen=lambda: W.selective_scan_inputs(host_shape, seed=0), keys=keys,
                    device_extra=lambda dev: dict(z=_device_normal((s.batch, s.dim, s.seqlen), dev, seed=0)),
                    call=lambda d: xp.selective_scan_fn(*(d[k] for k in keys), delta_softplus=True),
                    prepare=lambda d: xp.selective_scan_fn(*(d[k] for k in keys), delta_softplus=True, prepare=True),
                    tokens=s.batch * s.seqlen, nbytes=W.selective_scan_bytes(s),
                    config=dict(batch=s.batch, dim=s.dim, seqlen=s.seqlen, dstate=s.dstate, variable_B_C=True,
                                delta_softplus=True, has_D=True, has_z=True, has_delta_bias=True))

    def gdn2():
        s = W.GDN2_MAIN
        keys = ("q", "k", "v", "g", "beta", "w", "initial_state")
        return dict(name="gated_deltanet2", workload="gated_deltanet2_b4_t4096_h16_k128_v128", shape=s,
                    gen=lambda: W.gated_deltanet2_inputs(s, seed=0), keys=keys,
                    call=lambda d: xp.gated_deltanet2_fn(*(d[k] for k in keys), scale=s.scale),
                    prepare=lambda d: xp.gated_deltanet2_fn(*(d[k] for k in keys), scale=s.scale, prepare=True),
                    tokens=s.batch * s.seqlen, nbytes=W.gated_deltanet2_bytes(s),
                    config=dict(batch=s.batch, seqlen=s.seqlen, nheads=s.nheads, dk=s.dk, dv=s.dv,
                                initial_state=True, l2norm=True))

    def m3():
        s = W.M3_MAIN
        keys = ("Q", "K", "V", "ADT", "DT", "Trap", "Q_bias", "K_bias", "Angles", "D", "Z")
        return dict(name="mamba3_siso", workload="mamba3_siso_b4_t4096_h32_p64_n128", shape=s,
                    gen=lambda: W.mamba3_siso_inputs(s, seed=0), keys=keys,
                    call=lambda d: xp.mamba3_siso_fn(*(d[k] for k in keys)),
                    prepare=lambda d: xp.mamba3_siso_fn(*(d[k] for k in keys), prepare=True),
                    tokens=s.batch * s.seqlen, nbytes=W.mamba3_siso_bytes(s),
                    config=dict(batch=s.batch, seqlen=s.seqlen, nheads=s.nheads, headdim=s.headdim,
                                dstate=s.dstate, angles=s.a, has_d=True, has_z=False))

    return {"selective_scan": ss, "gated_deltanet2": gdn2, "mamba3_siso": m3}


def _device_normal(shape, dev, seed):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return torch.randn(shape, generator=g, device=dev, dtype=torch.float32)


def to_device(inputs, dev):
    import numpy as np
    import torch
    return {k: (None if v is None else torch.from_numpy(np.ascontiguousarray(v)).to(dev)) for k, v in inputs.items()}


def time_op(op, dev_inputs, steps, warmup, settle_ms=0.0):
    """Per-call HIP-event times (ms) on the current stream and the wall time of
    the `steps` timed calls.  Ops with a "prepare" entry are timed through a
    PreparedCall (argument blocks built once, the same C entry point and
    kernels per call), so a call of a few microseconds is not timed behind the
    Python front end's per-call descriptor work."""
    import torch
    if "prepare" in op:
        prepared = op["prepare"](dev_inputs)
        call = lambda: prepared()
    else:
        call = lambda: op["call"](dev_inputs)
    end = time.perf_counter() + settle_ms / 1e3
    while time.perf_counter() < end:   # untimed: the clock settles under this load
        for _ in range(8):
            call()
        torch.cuda.synchronize()
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for a, b in ev:
        a.record()
        call()
        b.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [a.elapsed_time(b) for a, b in ev]
    return wall, per


def probe_lib():
    """The HBM streaming probe (csrc/probe/hbm_stream.hip, libxm_hbm_probe.so)."""
    import ctypes
    from xmetai_onnx_plugins import _capi
    path = os.path.join(os.path.dirname(_capi.LIB_PATH), "libxm_hbm_probe.so")
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build with `python xmetai-onnx-plugins_amd/build.py`")
    lib = ctypes.CDLL(path)
    for fn in (lib.xm_probe_hbm_copy, lib.xm_probe_hbm_read):
        fn.restype = ctypes.c_int
    lib.xm_probe_hbm_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_void_p]
    lib.xm_probe_hbm_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_void_p]
    return lib


def achievable_hbm(dev, gib=2, reps=5):
    """Achievable HBM bandwidth from the hand-written streaming kernels of
    libxm_hbm_probe.so over `gib` GiB buffers: a copy (read + write, bytes
    counted both ways) and a read-only pass.  Sweeps workgroups per CU (4-32),
    16-byte vectors in flight per thread (1-8) and the nontemporal policy; each
    configuration takes the best of `reps` timed runs after one warm-up, and
    the best configuration is reported.  HIP events on the launch stream."""
    import ctypes
    import torch
    lib = probe_lib()
    nbytes = gib << 30
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.zeros(cus * 32, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)

    def timed(fn):
        best = float("inf")
        fn()
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            fn()
            b.record(stream)
            b.synchronize()
            best = min(best, a.elapsed_time(b))
        return best

    res = {}
    for kind in ("copy", "read"):
        top = (0.0, None)
        for per_cu in (4, 8, 16, 32):
            for unroll in (1, 2, 4, 8):
                for nt in (0, 1):
                    blocks = cus * per_cu
                    if kind == "copy":
                        fn = lambda: lib.xm_probe_hbm_copy(src.data_ptr(), dst.data_ptr(), nbytes, blocks, unroll, nt, sp)
                        moved = 2 * nbytes
                    else:
                        fn = lambda: lib.xm_probe_hbm_read(src.data_ptr(), nbytes, sink.data_ptr(), blocks, unroll, nt, sp)
                        moved = nbytes
                    if fn() != 0:
                        raise RuntimeError(f"HBM probe {kind} launch failed")
                    gbps = moved / (timed(fn) / 1e3) / 1e9
                    if gbps > top[0]:
                        top = (gbps, dict(workgroups_per_cu=per_cu, vectors_in_flight=unroll, nontemporal=nt))
        res[kind] = top
    del src, dst, sink
    torch.cuda.empty_cache()
    return dict(copy_GBps=round(res["copy"][0], 1), copy_config=res["copy"][1], read_GBps=round(res["read"][0], 1),
                read_config=res["read"][1], buffer_GiB=gib)


# ---------------------------------------------------------------------------
# CPU baseline (reference CPU path: NumPy fp32 sequential recurrences)
# ---------------------------------------------------------------------------

def cpu_env():
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count()
    return dict(host_cores_available=cores, OMP_NUM_THREADS=os.environ.get("OMP_NUM_THREADS"),
                OPENBLAS_NUM_THREADS=os.environ.get("OPENBLAS_NUM_THREADS"))


def cpu_baseline(op, inputs, budget_s):
    """Times the NumPy fp32 oracle on a slice of the workload that finishes in
    about `budget_s` seconds and scales to the full workload (cost is linear in
    the sliced axis).  NumPy's elementwise loops run on one core."""
    import numpy as np
    from oracle import numpy_ref

    s = op["shape"]
    name = op["name"]

    if name == "selective_scan":
        full_units = s.batch * s.dim

        def run(n):
            # n (batch, channel) pairs: channels of batch 0, or whole batches
            nb = -(-n // s.dim)
            nch = n if nb == 1 else s.dim
            sub = {k: inputs[k] for k in op["keys"]}
            for k in ("u", "delta"):
                sub[k] = np.ascontiguousarray(inputs[k][:nb, :nch])
            for k in ("A", "D", "delta_bias"):
                sub[k] = np.ascontiguousarray(inputs[k][:nch])
            sub["B"] = np.ascontiguousarray(inputs["B"][:nb])
            sub["C"] = np.ascontiguousarray(inputs["C"][:nb])
            sub["z"] = None
            t = time.perf_counter()
            numpy_ref.selective_scan(**sub, delta_softplus=True, dtype=np.float32)
            return time.perf_counter() - t, nb * nch

        unit = "(batch, channel) pairs"
        sample_fmt = ("{n} of {full} (batch, channel) pairs x {L} tokens, dstate {N} (NumPy fp32 oracle), "
                      "scaled by pair count")
        fmt_args = dict(L=s.seqlen, N=s.dstate)
    else:
        full_units = s.batch * s.nheads

        def run(n):
            # n (batch, head) pairs: heads of batch 0, or whole batches
            nb = -(-n // s.nheads)
            nh = n if nb == 1 else s.nheads
            sub = {}
            for k in op["keys"]:
                v = inputs[k]
                if v is None:
                    sub[k] = None
                elif k in ("ADT", "DT", "Trap", "initial_state"):
                    sub[k] = np.ascontiguousarray(v[:nb, :nh])
                elif k in ("Q_bias", "K_bias", "D"):
                    sub[k] = np.ascontiguousarray(v[:nh])
                else:
                    sub[k] = np.ascontiguousarray(v[:nb, :, :nh])
            t = time.perf_counter()
            if name == "gated_deltanet2":
                numpy_ref.gated_deltanet2(*(sub[k] for k in op["keys"]), scale=s.scale, dtype=np.float32)
            else:
                numpy_ref.mamba3_siso(*(sub[k] for k in op["keys"]), dtype=np.float32)
            return time.perf_counter() - t, nb * nh

        unit = "(batch, head) pairs"
        sample_fmt = "{n} of {full} (batch, head) pairs x {T} tokens (NumPy fp32 oracle), scaled by pair count"
        fmt_args = dict(T=s.seqlen)
    max_units = full_units

    # calibrate on growing slices until one takes >= 0.5 s, then size the
    # measured slice to the budget
    n = 1
    t, n = run(n)
    while t < 0.5 and n < max_units:
        t, n = run(min(max_units, n * 4))
    if t < budget_s * 0.8 and n < max_units:
        t, n = run(min(max_units, max(n + 1, int(n * budget_s / max(t, 1e-3)))))
    t_full = t * full_units / n
    tokens = op["tokens"]
    return dict(value=tokens / t_full, unit="tokens/s", cores=1, kind="port",
                sample=sample_fmt.format(n=n, full=full_units, **fmt_args), sample_seconds=round(t, 3),
                sampled_units=n, unit_axis=unit, **cpu_env())


# ---------------------------------------------------------------------------

def named_op(name):
    """A named workload of the CPU-sized selective scan or a GDN-2 dispatch
    boundary as a prepared call: (host inputs, prepare, algorithmic bytes, tokens)."""
    from xmetai_onnx_plugins import workloads as W
    import xmetai_onnx_plugins as xp
    s = W.NAMED[name]
    if name.startswith("selective_scan"):
        keys = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
        inp = W.selective_scan_inputs(s, seed=0)
        prep = lambda d: xp.selective_scan_fn(*(d[k] for k in keys), delta_softplus=s.delta_softplus, prepare=True)
        nbytes = W.selective_scan_bytes(s)
    elif name.startswith("gated_deltanet2"):
        keys = ("q", "k", "v", "g", "beta", "w", "initial_state")
        inp = W.gated_deltanet2_inputs(s, seed=0)
        prep = lambda d: xp.gated_deltanet2_fn(*(d[k] for k in keys), scale=s.scale, prepare=True)
        nbytes = W.gated_deltanet2_bytes(s)
    else:
        raise SystemExit(f"no prepared form for workload {name}")
    return inp, prep, nbytes, s.batch * s.seqlen


EXTRA_CONFIGS = ("selective_scan_b1_d256_l512_n16", "gated_deltanet2_b1_t16384_h8_k256_v256",
                 "gated_deltanet2_b2_t2048_h4_k320_v64", "gated_deltanet2_b4_t4096_h16_k128_v65")


def time_extra_configs(dev, steps, settle_ms):
    """The reference's other configurations (CPU-sized selective scan, GDN-2
    dispatch boundaries): device time only, same inputs and timing as above."""
    import torch
    import xmetai_onnx_plugins as xp
    out = {}
    for name in EXTRA_CONFIGS:
        inp, prep, nbytes, tokens = named_op(name)
        d = to_device(inp, dev)
        _, per = time_op(dict(prepare=prep), d, steps, 2, settle_ms)
        kernels = xp.last_launches()
        ms = statistics.median(per)
        out[name] = dict(ms_per_call_median=round(ms, 4), tokens_per_s=tokens / (ms / 1e3),
                         achieved_GBps=round(nbytes / (ms / 1e3) / 1e9, 1), algorithmic_bytes=nbytes,
                         kernels=kernels)
        log(f"{name}: {ms:.3f} ms/call")
        del d, inp
        torch.cuda.empty_cache()
    return out


def traffic_from_profiles(workload):
    path = os.path.join(ROOT, "profiles", f"{workload}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--settle-ms", type=float, default=500.0,
                    help="untimed calls of each operator for this long before its warmup steps")
    ap.add_argument("--ops", default="selective_scan,gated_deltanet2,mamba3_siso")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU-baseline budget per op (seconds)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra-configs", action="store_true",
                    help="skip timing the other reference configurations (reported under 'configs')")
    ap.add_argument("--override", action="append", default=[], metavar="NAME=VALUE",
                    help="profile modes only: force a kernel variant (xm_set_kernel_override), e.g. gdn2_path=1")
    ap.add_argument("--mode", default="bench",
                    help="bench | copy | profile-selective_scan | profile-gated_deltanet2 | profile-mamba3_siso | "
                         "profile-<workload> for one of the other configurations (" + ", ".join(EXTRA_CONFIGS) + ")")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: the operators are single-GPU ORT kernels with no "
              "collectives; --gpus above 1 is not supported (multi-GPU sharding is design-only).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.mode == "copy":
        # counter calibration: the probe's copy kernel over 1 GiB, three times
        import ctypes
        lib = probe_lib()
        n = (1 << 30) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        sp = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        for _ in range(3):
            if lib.xm_probe_hbm_copy(src.data_ptr(), dst.data_ptr(), n * 4, 256 * 8, 4, 0, sp) != 0:
                raise RuntimeError("HBM probe copy launch failed")
        torch.cuda.synchronize()
        log("copied 1 GiB x 3 (HbmCopyKernel<4,false>)")
        return

    import xmetai_onnx_plugins as xp
    if args.override and not args.mode.startswith("profile-"):
        raise SystemExit("--override applies to the profile modes only")
    builders = make_ops()
    if args.mode.startswith("profile-"):
        name = args.mode[len("profile-"):]
        for ov in args.override:
            key, _, val = ov.partition("=")
            xp.set_kernel_override(key, int(val))
        if name in builders:
            op = builders[name]()
            d = to_device(op["gen"](), dev)
            if "device_extra" in op:
                d.update(op["device_extra"](dev))
        else:   # one of the other configurations, by workload name
            inp, prep, _, _ = named_op(name)
            op, d = dict(prepare=prep), to_device(inp, dev)
        wall, per = time_op(op, d, args.steps, args.warmup, args.settle_ms)
        log(f"{name}: {statistics.median(per):.3f} ms/call (median of {args.steps})")
        return

    names = [n for n in args.ops.split(",") if n]
    if "selective_scan" not in names:
        names.insert(0, "selective_scan")
    results = {}
    headline = None
    for name in names:
        op = builders[name]()
        log(f"{name}: generating {op['workload']}")
        host = op["gen"]()
        d = to_device(host, dev)
        if "device_extra" in op:
            d.update(op["device_extra"](dev))
        torch.cuda.synchronize()
        log(f"{name}: timing {args.settle_ms:.0f} ms settle + {args.warmup} warmup + {args.steps} steps")
        wall, per = time_op(op, d, args.steps, args.warmup, args.settle_ms)
        kernels = xp.last_launches()   # the dispatch the timed calls took
        ev_ms = sum(per) / len(per)
        med_ms = statistics.median(per)
        gbps = op["nbytes"] / (med_ms / 1e3) / 1e9
        r = dict(workload=op["workload"], config=op["config"], tokens_per_call=op["tokens"],
                 ms_per_call_median=round(med_ms, 4), ms_per_call_mean=round(ev_ms, 4),
                 tokens_per_s=op["tokens"] / (med_ms / 1e3), algorithmic_bytes=op["nbytes"],
                 achieved_GBps=round(gbps, 1), frac_hbm_peak=round(gbps / HBM_PEAK_GBPS, 4), kernels=kernels)
        # the form that runs: GDN-2 at head_k <= 256 is the chunked MFMA form
        fl = floors_us(name, op["shape"], op["nbytes"])
        binding = max((k for k in fl if k != "valu_sequential_form"), key=lambda k: fl[k])
        r.update(floors_us=fl, binding_floor=binding, frac_of_binding_floor=round(fl[binding] / (med_ms * 1e3), 4))
        log(f"{name}: {med_ms:.3f} ms/call, {r['tokens_per_s']:.4g} tokens/s, {gbps:.0f} GB/s")
        if not args.no_cpu_baseline:
            budget = args.cpu_seconds
            log(f"{name}: CPU baseline (~{budget:.0f} s)")
            r["cpu_baseline"] = cpu_baseline(op, host, budget)
            log(f"{name}: CPU {r['cpu_baseline']['value']:.4g} tokens/s ({r['cpu_baseline']['sample']})")
        results[name] = r
        if name == "selective_scan":
            headline = dict(wall=wall, per=per, op=op)
        del d, host
        torch.cuda.empty_cache()

    extra = {} if args.no_extra_configs else time_extra_configs(dev, min(args.steps, 20), min(args.settle_ms, 200.0))

    log("achievable HBM: streaming-kernel sweep over 2 GiB buffers")
    probe = achievable_hbm(dev)
    ach = probe["copy_GBps"]
    log(f"achievable HBM: copy {ach} GB/s {probe['copy_config']}, read {probe['read_GBps']} GB/s")
    for r in results.values():
        r["frac_achievable_hbm"] = round(r["achieved_GBps"] / ach, 4)

    op = headline["op"]
    steps = args.steps
    wall = headline["wall"]
    ev_avg_ms = sum(headline["per"]) / len(headline["per"])
    achieved = op["nbytes"] / (ev_avg_ms / 1e3) / 1e9
    ss = results["selective_scan"]
    line = {
        "metric": METRIC,
        "value": op["tokens"] * steps / wall,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "settle_ms": args.settle_ms,
        "ms_per_step": wall * 1e3 / steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded NumPy draws with the reference configs' distributions, resident in HBM",
        "config": dict(workload=op["workload"], **op["config"]),
        # bound: the roofline the fraction is taken against.  The selective scan
        # has no dense contraction (no MFMA roofline), so it is HBM; its
        # binding compute floor (non-packed VALU issue) is reported beside it.
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic_from_profiles(op["workload"]),
            "kernel": ";".join(ss["kernels"]),
            "algorithmic_bytes_per_launch": op["nbytes"],
            "kernel_ms_avg": round(ev_avg_ms, 4),
            "frac_of_achievable": round(achieved / ach, 4),
            "achievable": ach,
            "floors_us": ss["floors_us"],
            "binding_floor": ss["binding_floor"],
            "frac_of_binding_floor": round(ss["floors_us"][ss["binding_floor"]] / (ev_avg_ms * 1e3), 4),
        },
        "cpu_baseline": ss.get("cpu_baseline"),
        "achievable_hbm_GBps": ach,
        "hbm_probe": probe,
        "ops": results,
        "configs": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
