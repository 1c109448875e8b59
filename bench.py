"""Benchmark of the adapter-augmented layer hot path on one MI355X.

One step = route the batch's tokens on the device (router features -> priors -> Q15 rings) and run
the int4 SwiGLU MLP with each token's K LoRA adapters (shrink, fused int4 GEMV + expand + SwiGLU,
shrink, down GEMV + expand). The headline workload is the Qwen2.5-7B-shaped decode step at one
token (hidden 3584, intermediate 18944, 16 adapters of rank 16, K = 4); the same line reports the
8-token decode batch and the 2048-token prefill with its MFMA utilisation, the roofline of the
dominant kernel (live per-kernel times from dispatch-recorded HIP events) and the CPU baseline
(the C oracle on this host's cores, a bounded sample).

The line also carries the token decode of a whole Qwen2.5-7B-shaped model (embedding, 28 decoder
layers with attention over a 512-token KV cache, LM head) through aoship_model_forward.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu] [--skip-prefill] [--skip-model]
       python bench.py --probe | --probe-prefill   (workloads for the hardware-counter runs)
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "adapter-os_amd"))

METRIC = "decode tok/s + HBM GB/s; prefill MFMA util — Qwen7B-shape int4 SwiGLU+K=4 LoRA"
HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class MlpCase:
    """Device-resident layers, router and inputs for T tokens of a workload.

    n_layers distinct copies of the layer (own int4 weights and own LoRA weights per layer, as
    consecutive transformer layers have) are cycled step by step, so that every step streams its
    weights from HBM: one 7B-shaped layer (123 MB) would otherwise stay resident in the 256 MB
    last-level cache across back-to-back calls."""

    def __init__(self, aoship, W, cid: int, T: int, torch, n_layers: int = 1):
        self.cfg = cfg = W.CONFIGS[cid]
        self.T = T
        self.torch = torch
        self.n_layers = n_layers
        base = {m: W.base_weights(cfg, m) for m in cfg.modules}
        self.adapters = []
        for a in range(cfg.n_adapters):
            ad = aoship.LoraAdapter(a, n_layers, W.lora_scale(cfg))
            for m in cfg.modules:
                A, B = W.lora_weights(cfg, a, m)
                for li in range(n_layers):
                    ad.set_module(li, m, A, B)
            self.adapters.append(ad)
        self.layers = []
        for li in range(n_layers):
            layer = aoship.Layer(li)
            for m in cfg.modules:
                p, s, b = base[m]
                layer.set_base(m, p, s, b)
            layer.set_adapters(self.adapters)
            layer.reserve(T)
            self.layers.append(layer)
        del base
        sid = np.arange(cfg.n_adapters, dtype=np.uint64)
        self.router = aoship.Router(cfg.n_adapters, cfg.k, cfg.tau, cfg.eps, 1.0, sid)
        xb, _ = W.activations(cfg, T)
        self.x = torch.from_numpy(xb.view(np.int16)).cuda()
        self.y = torch.empty((T, cfg.hidden), dtype=torch.int16, device="cuda")
        self.rings = torch.zeros(T * 40, dtype=torch.uint8, device="cuda")
        if cfg.routing == "features":
            f, w = W.router_inputs(cfg, T)
            self.f = torch.from_numpy(f).cuda()
            self.w = torch.from_numpy(w).cuda()
            self.priors = None
        else:
            self.priors = torch.from_numpy(W.priors(cfg, T)).cuda()
        self.i = 0
        self.combined = False  # route and MLP in one call (aoship_route_mlp_forward)

    def step(self):
        if self.combined and self.priors is None:
            self.layers[self.i % self.n_layers].route_mlp_forward(self.router, self.f, self.w, self.x, self.rings,
                                                                   self.y)
            self.i += 1
            return
        if self.priors is None:
            self.router.route_features(self.f, self.w, self.rings)
        else:
            self.router.route(self.priors, self.rings)
        self.layers[self.i % self.n_layers].mlp_forward(self.x, self.rings, self.y)
        self.i += 1

    def check_waits(self):
        """A fused launch whose bounded wait gave up returns early with invalid output: a timed
        block with one is not a valid measurement."""
        self.torch.cuda.synchronize()
        bad = [i for i, layer in enumerate(self.layers) if layer.wait_timeouts() != 0]
        if bad:
            raise RuntimeError(f"a fused launch gave up waiting on layer copies {bad}: the timing is invalid")

    def set_profiling(self, on: bool):
        for layer in self.layers:
            layer.set_profiling(on)

    def kernel_stats(self) -> dict:
        tot = {}
        for layer in self.layers:
            for k, (ms, n) in layer.kernel_stats().items():
                a, b = tot.get(k, (0.0, 0))
                tot[k] = (a + ms, b + n)
        return tot

    def distinct_adapters(self, aoship) -> int:
        self.torch.cuda.synchronize()
        r = aoship.rings_from_bytes(self.rings.cpu().numpy())
        used = set()
        for t in range(len(r)):
            k = int(r[t]["top_k"])
            for s in range(k):
                if r[t]["gates_q15"][s] > 0:
                    used.add(int(r[t]["adapter_indices"][s]))
        return len(used)


class ProjCase:
    """Device-resident attention projections (q, k, v, o) of a workload for T concurrent decode
    streams, each token with its own routed adapter set: n_layers distinct copies of the layer
    (own int4 weights and LoRA weights) are cycled step by step so the weights stream from HBM.
    A step routes the T tokens from their features, then runs q/k/v in one call and o in another;
    with route=False the rings of the first routing are reused (the projections alone)."""

    def __init__(self, aoship, W, cid: int, T: int, torch, n_layers: int):
        self.cfg = cfg = W.CONFIGS[cid]
        self.T, self.torch, self.n_layers = T, torch, n_layers
        base = {m: W.base_weights(cfg, m) for m in cfg.modules}
        self.adapters = []
        for a in range(cfg.n_adapters):
            ad = aoship.LoraAdapter(a, n_layers, W.lora_scale(cfg))
            for m in cfg.modules:
                A, B = W.lora_weights(cfg, a, m)
                for li in range(n_layers):
                    ad.set_module(li, m, A, B)
            self.adapters.append(ad)
        self.layers = []
        for li in range(n_layers):
            layer = aoship.Layer(li)
            for m in cfg.modules:
                p, sc, b = base[m]
                layer.set_base(m, p, sc, b)
            layer.set_adapters(self.adapters)
            layer.reserve(T)
            self.layers.append(layer)
        del base
        sid = np.arange(cfg.n_adapters, dtype=np.uint64)
        self.router = aoship.Router(cfg.n_adapters, cfg.k, cfg.tau, cfg.eps, 1.0, sid)
        xb, _ = W.activations(cfg, T)
        self.x = torch.from_numpy(xb.view(np.int16)).cuda()
        self.xo = torch.from_numpy(W.activations(cfg, T, cfg.q_out)[0].view(np.int16)).cuda()
        self.q = torch.empty((T, cfg.q_out), dtype=torch.int16, device="cuda")
        self.k = torch.empty((T, cfg.kv_out), dtype=torch.int16, device="cuda")
        self.v = torch.empty((T, cfg.kv_out), dtype=torch.int16, device="cuda")
        self.o = torch.empty((T, cfg.hidden), dtype=torch.int16, device="cuda")
        self.rings = torch.zeros(T * 40, dtype=torch.uint8, device="cuda")
        f, w = W.router_inputs(cfg, T)
        self.f = torch.from_numpy(f).cuda()
        self.w = torch.from_numpy(w).cuda()
        self.router.route_features(self.f, self.w, self.rings)
        self.route = True
        self.i = 0

    def step(self):
        if self.route:
            self.router.route_features(self.f, self.w, self.rings)
        layer = self.layers[self.i % self.n_layers]
        layer.qkv_forward(self.x, self.rings, self.q, self.k, self.v)
        layer.proj_forward("o_proj", self.xo, self.rings, self.o)
        self.i += 1

    check_waits = MlpCase.check_waits
    set_profiling = MlpCase.set_profiling
    kernel_stats = MlpCase.kernel_stats
    distinct_adapters = MlpCase.distinct_adapters


class RouteOnly:
    """A case's router launch alone (priors or features, as the case routes)."""

    def __init__(self, case):
        self.case = case

    def step(self):
        c = self.case
        if c.priors is None:
            c.router.route_features(c.f, c.w, c.rings)
        else:
            c.router.route(c.priors, c.rings)

    def check_waits(self):
        pass


def time_steps(case, steps: int, warmup: int, torch) -> float:
    """Milliseconds per step over `steps` steps, events on the launch stream (the null stream). The
    warm-up covers every layer copy a case cycles through at least once."""
    for _ in range(max(warmup, getattr(case, "n_layers", 0))):
        case.step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        case.step()
    end.record()
    torch.cuda.synchronize()
    case.check_waits()
    return start.elapsed_time(end) / steps


def kernel_times(case, steps: int, torch) -> dict:
    """Average per-launch kernel durations (ms) from events the dispatches record."""
    case.set_profiling(True)
    for _ in range(steps):
        case.step()
    torch.cuda.synchronize()
    case.check_waits()
    st = case.kernel_stats()
    case.set_profiling(False)
    return {k: ms / n for k, (ms, n) in st.items() if n}


# The decode shrinks run in the first workgroups of the GEMV launch that reads their S.
FUSED = True


def c4_bytes(cfg, T: int, U: int) -> int:
    """Algorithmic HBM bytes of one C4 step's projections: the int4 q/k/v/o matrices with their f16
    scales and biases, the bf16 LoRA A and B rows of the U distinct adapters on all four, and the
    bf16 activations (x in, q/k/v out, o's input in, o out)."""
    base = lora = 0
    for m in cfg.modules:
        out, inp = cfg.shape(m)
        base += out * inp // 2 + 2 * 2 * out * (inp // 64)
        lora += cfg.rank * (inp + out) * 2
    acts = T * cfg.hidden * 2 + T * (cfg.q_out + 2 * cfg.kv_out) * 2 + T * cfg.q_out * 2 + T * cfg.hidden * 2
    return base + U * lora + acts


def gate_up_bytes(cfg, T: int, U: int) -> int:
    """Algorithmic HBM bytes of one gate/up launch: both int4 matrices with their f16 scale and
    bias, the bf16 LoRA B rows of the U distinct adapters for both modules, x in and h out; with
    the x shrink in the same launch also the U adapters' bf16 A rows for both modules (the shrink
    reads every bound adapter's rows when that is cheaper than waiting for the plan: the excess
    is traffic above the algorithmic bytes), and at 1 or 2 tokens the U adapters' A_down rows,
    whose products with h this launch forms for the down projection's shrink."""
    H, I = cfg.hidden, cfg.inter
    base = 2 * (I * H // 2 + 2 * 2 * I * (H // 64))
    lora = U * 2 * I * cfg.rank * 2 + (U * 2 * cfg.rank * H * 2 if FUSED else 0)
    if FUSED and T <= 2:
        lora += U * cfg.rank * I * 2
    return base + lora + T * H * 2 + T * I * 2


def launch_names(kt: dict, combined: bool = False) -> dict:
    """Per-launch times keyed by what each launch runs (a fused shrink has no launch of its own;
    with the combined call the router runs in the gate/up launch)."""
    if not FUSED:
        return dict(kt)
    gu = ("route+" if combined else "") + "lora_shrink_x+q4_gemv_gate_up"
    ren = {"q4_gemv_gate_up": gu, "q4_gemv_down": "lora_shrink_h+q4_gemv_down",
           "mlp1": ("route+" if combined else "") + "mlp1"}
    return {ren.get(k, k): v for k, v in kt.items() if k not in ("lora_shrink_x", "lora_shrink_h")}


PROFILES = ROOT / "profiles"
TRAFFIC_FILE = PROFILES / "q4_gemv_gate_up__qwen7b_decode_t1__hbm_traffic.md"
MLP1_TRAFFIC_FILE = PROFILES / "mlp1__qwen7b_decode_t1__hbm_traffic.md"
COPY_BYTES = 512 << 20


def probe(aoship, W, torch, layers: int) -> int:
    """Workload for the hardware-counter runs (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE): 50 decode
    steps of the headline workload (1 token, one aoship_route_mlp_forward call per step), 50 of the
    same token as two calls (route, then the MLP), 50 of the 8-token batch, 48 steps of the C4
    projections (32 streams, rings given), then one device copy of COPY_BYTES that calibrates the
    counters (it reads and writes exactly COPY_BYTES). Each workload's launches have kernel
    instances or grids of their own."""
    for T, combined in ((1, True), (1, False), (8, False)):
        dec = MlpCase(aoship, W, 2, T, torch, layers)
        dec.combined = combined
        for _ in range(50):
            dec.step()
        torch.cuda.synchronize()
        del dec
    c4 = ProjCase(aoship, W, 4, 32, torch, 24)
    c4.route = False
    for _ in range(48):
        c4.step()
    torch.cuda.synchronize()
    del c4
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    log("probe done")
    return 0


def probe_prefill(aoship, W, torch) -> int:
    """Workload for the prefill counter runs: 6 steps of the 2048-token prefill (C3), then 3 of the
    4096-token stress prefill (C5, whose GEMMs run as stream-K and whose tile shrinks are launches of
    their own, so its launches are told apart by kernel and grid)."""
    for cid, T, n in ((3, 2048, 6), (5, 4096, 3)):
        pf = MlpCase(aoship, W, cid, T, torch, 1)
        for _ in range(n):
            pf.step()
        torch.cuda.synchronize()
        del pf
    log("prefill probe done")
    return 0


def measured_mfma_peak() -> float | None:
    """Achievable dense bf16 MFMA TFLOP/s on this GPU (chains of v_mfma_f32_32x32x16_bf16 on every
    SIMD, no memory traffic), from the probe library the build compiles; None when absent."""
    import ctypes

    path = ROOT / "adapter-os_amd" / "libaos_peak.so"
    if not path.exists():
        return None
    lib = ctypes.CDLL(str(path))
    lib.aos_mfma_peak_tflops.restype = ctypes.c_double
    lib.aos_mfma_peak_tflops.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
    tf = lib.aos_mfma_peak_tflops(2048, 4096, 5)
    return tf if tf > 0 else None


def hbm_stream_probe(gate_up_b: int, down_b: int, layer_b: int) -> dict | None:
    """What one launch can read from HBM here (the probe library's stream kernel: the decode GEMVs'
    pattern of contiguous 1 KiB chunks per wave, 4-wave workgroups, each timed launch after a 1 GiB
    read that evicts the caches; median of 7 launches). Reports the ceiling (1 GiB, best of the
    workgroup counts and ring depths tried) and, for the byte counts of the decode launches, the
    best one-launch time and the time at the decode grids' workgroup counts; None when absent."""
    import ctypes

    path = ROOT / "adapter-os_amd" / "libaos_peak.so"
    if not path.exists():
        return None
    lib = ctypes.CDLL(str(path))
    fn = lib.aos_hbm_stream_us
    fn.restype = ctypes.c_double
    fn.argtypes = [ctypes.c_long, ctypes.c_int, ctypes.c_int, ctypes.c_int]

    def best(nbytes: int, wgs_list, depths=(4, 8)) -> dict:
        nbytes -= nbytes % 1024
        out = None
        for wgs in wgs_list:
            for d in depths:
                us = fn(nbytes, wgs, d, 7)
                if us <= 0:
                    raise RuntimeError("HBM stream probe failed")
                if out is None or us < out["us"]:
                    out = {"us": us, "tbps": nbytes / (us * 1e-6) / 1e12, "workgroups": wgs, "depth": d}
        out["bytes"] = nbytes
        return out

    grids = (256, 512, 768, 1024, 1536, 2048)
    res = {
        "ceiling": best(1 << 30, (1024, 2048, 4096, 8192)),
        "gate_up_bytes": best(gate_up_b, grids),
        "down_bytes": best(down_b, grids),
        "gate_up_bytes_at_592_workgroups": best(gate_up_b, (592,), (4,)),
        "down_bytes_at_448_workgroups": best(down_b, (448,), (4,)),
        "layer_bytes": best(layer_b, grids),
    }
    lib.aos_hbm_stream_free()
    res["two_launch_floor_us"] = res["gate_up_bytes"]["us"] + res["down_bytes"]["us"]
    res["note"] = ("plain streaming kernels, no compute: a lower bound for one launch per matrix; the "
                   "592- and 448-workgroup lines read the same bytes with the decode grids' workgroup "
                   "counts (592 row blocks of gate/up; 448 down workgroups); layer_bytes: the whole "
                   "layer's algorithmic bytes in one launch, the floor of the one-token launch")
    return res


def measured_traffic(path=TRAFFIC_FILE):
    """HBM bytes per launch of the headline kernel from its committed counter summary, or None."""
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def host_cpu_info() -> dict:
    """The host's CPU topology (lscpu), the logical CPUs the OS reports (nproc) and the CPUs this
    process may run on (its affinity mask)."""
    info = {"nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0))}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        out = ""
    keys = {"Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket", "Thread(s) per core": "threads_per_core",
            "Model name": "model"}
    for line in out.splitlines():
        k, _, v = line.partition(":")
        k = k.strip()
        if k in keys:
            v = v.strip()
            info[keys[k]] = int(v) if v.isdigit() else v
    if all(k in info for k in ("sockets", "cores_per_socket")):
        info["physical_cores"] = info["sockets"] * info["cores_per_socket"]
    return info


def cpu_baseline(W, T: int = 1, runs: int = 20) -> dict:
    """The C oracle (float32, dequantising on the fly, OpenMP over output rows) on this host, on the
    7B-shaped decode workload: the router (priors from features, then routing) and the layer (int4
    SwiGLU MLP with the K=4 LoRA deltas) timed separately, each the median of `runs` timed calls
    after warm-up, once on every CPU this job may use and once on one thread."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    cfg = W.CONFIGS[2]
    bw = {m: W.base_weights(cfg, m) for m in cfg.modules}
    lora = [{m: W.lora_weights(cfg, a, m) for m in cfg.modules} for a in range(cfg.n_adapters)]
    scales = np.full(cfg.n_adapters, W.lora_scale(cfg), np.float32)
    f, w = W.router_inputs(cfg, T)
    _, xf = W.activations(cfg, T)
    sid = np.arange(cfg.n_adapters, dtype=np.uint64)
    rings = None

    def router():
        nonlocal rings
        pri = oracle.priors(f, w)
        rings = oracle.route_batch(pri, cfg.k, cfg.tau, cfg.eps, 1.0, sid)

    def layer():
        oracle.mlp_forward(xf, bw["gate_proj"], bw["up_proj"], bw["down_proj"], lora, scales, cfg.rank, rings)

    def median_ms(fn) -> float:
        for _ in range(2):
            fn()
        times = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return float(np.median(times)) * 1e3

    host = host_cpu_info()
    # the CPUs this job may use: its affinity mask, or fewer when the job is given a thread budget
    # (OMP_NUM_THREADS; a GPU job here is allotted a share of the host's cores)
    threads = host["affinity_cpus"]
    budget = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    if budget > 0:
        threads = min(threads, budget)
    figures = {}
    for name, nt in (("all", threads), ("one", 1)):
        oracle.set_threads(nt)
        r_ms = median_ms(router)
        l_ms = median_ms(layer)
        figures[name] = {"threads": nt, "router_ms": r_ms, "layer_ms": l_ms, "tok_s": T / ((r_ms + l_ms) * 1e-3)}
    oracle.set_threads(threads)
    return {
        "value": figures["all"]["tok_s"],
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "sample": f"7B-shaped decode step, T={T}: router (features -> priors -> rings) and layer (int4 SwiGLU "
                  f"MLP + K=4 LoRA) each the median of {runs} timed calls after 2 warm-up calls; tok/s = T / "
                  f"(router + layer); on {threads} threads and on 1",
        "router_ms": figures["all"]["router_ms"],
        "layer_ms": figures["all"]["layer_ms"],
        "single_thread": figures["one"],
        "host": host,
        "threads_note": "threads = the CPUs in this process's affinity mask, capped by OMP_NUM_THREADS when set "
                        "(the CPU share a one-GPU job is given on a shared host)",
    }


def library_gemm_reference(torch, T: int, H: int, I: int) -> dict:
    """The vendor library's dense bfloat16 GEMM (torch.mm, hipBLASLt) on the prefill's shapes,
    with weights already in bfloat16 (no dequantisation, no LoRA, no SwiGLU): the gate and up
    projections as one [T, H] x [H, 2I] product, and down as [T, I] x [I, H]. A reference point
    for the int4 kernels, not part of the path."""
    out = {}
    for name, (m, k, n) in (("gate_up", (T, H, 2 * I)), ("down", (T, I, H))):
        a = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
        b = torch.randn(n, k, device="cuda", dtype=torch.bfloat16)
        for _ in range(3):
            torch.mm(a, b.t())
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            torch.mm(a, b.t())
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / 10 * 1e3
        out[name] = {"us": us, "tflops": 2 * m * k * n / (us * 1e-6) / 1e12}
        del a, b
    return out


def model_decode(aoship, W, torch, n_layers: int, ctx: int, steps: int, warmup: int) -> dict:
    """Token decode of a Qwen2.5-7B-shaped model through aoship_model_forward: n_layers decoder
    layers (hidden 3584, intermediate 18944, 28 query and 4 key-value heads of 128, rope theta 1e6,
    vocab 152064, q/k/v biases), each with its own int4 weights on the device (four generated sets
    reused on the host), 16 rank-16 adapters on all seven projections, the token routed (K=4) by
    the device router before each step. The KV cache is first filled with ctx - 1 tokens by one
    prefill call; then each timed step routes one token and runs the whole model for it."""
    import dataclasses

    mlp = W.CONFIGS[2]
    attn = W.Config(6, "qwen7b-attn", "attn", mlp.hidden, q_out=3584, kv_out=512, n_adapters=mlp.n_adapters,
                    rank=mlp.rank, k=mlp.k, modules=("q_proj", "k_proj", "v_proj", "o_proj"))
    H, I, vocab, nh, nkv, hd = mlp.hidden, mlp.inter, 152064, 28, 4, 128
    max_seq = ctx + warmup + steps + 8
    model = aoship.Model(n_layers, H, I, nh, nkv, hd, vocab, max_seq, 1.0e6, 1e-6)
    sets = []
    for j in range(4):
        mc, ac = dataclasses.replace(mlp, cid=100 + j), dataclasses.replace(attn, cid=200 + j)
        sets.append({**{m: W.base_weights(mc, m) for m in mc.modules}, **{m: W.base_weights(ac, m) for m in ac.modules}})
    rng = np.random.default_rng(0xAD05)
    emb = (rng.integers(0, 2 ** 32, (vocab, H // 8), dtype=np.uint32),
           (rng.standard_normal((vocab, H // 64)) * 0.02).astype(np.float16),
           (rng.standard_normal((vocab, H // 64)) * 0.01).astype(np.float16))
    model.set_embedding(*emb)
    model.set_lm_head(*emb)
    bias = {m: (rng.standard_normal(n) * 0.02).astype(np.float32) for m, n in (("q_proj", nh * hd), ("k_proj", nkv * hd),
                                                                                ("v_proj", nkv * hd))}
    for li in range(n_layers):
        for m, w in sets[li % 4].items():
            model.layers[li].set_base(m, *w)
        for m, b in bias.items():
            model.set_bias(li, m, b)
    del sets
    adapters = []
    for a in range(mlp.n_adapters):
        ad = aoship.LoraAdapter(a, n_layers, W.lora_scale(mlp))
        for cfg in (mlp, attn):
            for m in cfg.modules:
                A, B = W.lora_weights(cfg, a, m)
                for li in range(n_layers):
                    ad.set_module(li, m, A, B)
        adapters.append(ad)
    model.set_adapters(adapters)
    model.reserve(ctx)
    router = aoship.Router(mlp.n_adapters, mlp.k, mlp.tau, mlp.eps, 1.0, np.arange(mlp.n_adapters, dtype=np.uint64))
    f, rw = W.router_inputs(mlp, ctx + warmup + steps)
    f, rw = torch.from_numpy(f).cuda(), torch.from_numpy(rw).cuda()
    ids = torch.from_numpy(rng.integers(0, vocab, ctx + warmup + steps).astype(np.int32)).cuda()
    rings = torch.zeros((ctx + warmup + steps) * 40, dtype=torch.uint8, device="cuda")
    logits = torch.empty(vocab, dtype=torch.float32, device="cuda")
    n0 = ctx - 1
    router.route_features(f[:n0], rw, rings[: n0 * 40])
    model.forward(ids[:n0], rings[: n0 * 40], logits)
    torch.cuda.synchronize()

    def step(i):
        router.route_features(f[i:i + 1], rw, rings[i * 40:(i + 1) * 40])
        model.forward(ids[i:i + 1], rings[i * 40:(i + 1) * 40], logits)

    for i in range(n0, n0 + warmup):
        step(i)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(n0 + warmup, n0 + warmup + steps):
        step(i)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    assert bool(torch.isfinite(logits).all())
    if any(layer.wait_timeouts() != 0 for layer in model.layers):
        raise RuntimeError("a fused launch of the model gave up waiting: the timing is invalid")
    # per layer: int4 weights + f16 scales/biases and the K routed adapters' bf16 rows of all seven
    # projections, and the bf16 keys and values of the (average) context; then the LM head
    layer_w = W.algorithmic_bytes(mlp, 1, mlp.k) + W.algorithmic_bytes(attn, 1, attn.k)
    kv = 2 * nkv * hd * 2 * (ctx + warmup + steps // 2)
    lm = vocab * H // 2 + vocab * (H // 64) * 4
    bytes_tok = n_layers * (layer_w + kv) + lm
    del model, adapters
    return {
        "workload": f"Qwen2.5-7B-shaped decoder, {n_layers} layers, 28/4 heads of 128, vocab 152064, int4 g64, "
                    f"16 rank-16 adapters on all projections, K=4 routed per token, context {ctx}",
        "layers": n_layers, "context": ctx, "steps": steps,
        "ms_per_token": ms, "tok_s": 1.0 / (ms * 1e-3),
        "approx_hbm_bytes_per_token": bytes_tok, "approx_hbm_gbps": bytes_tok / (ms * 1e-3) / 1e9,
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-prefill", action="store_true")
    ap.add_argument("--probe", action="store_true",
                    help="run the hardware-counter workload only (see probe())")
    ap.add_argument("--probe-prefill", action="store_true",
                    help="run the prefill hardware-counter workload only (see probe_prefill())")
    ap.add_argument("--skip-model", action="store_true", help="skip the full-model decode line")
    ap.add_argument("--skip-c4", action="store_true", help="skip the multi-tenant projection line (C4)")
    ap.add_argument("--skip-c5", action="store_true", help="skip the 32B stress prefill line (C5)")
    ap.add_argument("--probe-model", action="store_true",
                    help="run the full-model decode only (--model-layers layers) and print its figures")
    ap.add_argument("--model-layers", type=int, default=28)
    ap.add_argument("--layers", type=int, default=4,
                    help="distinct layer copies cycled by the decode steps (defeats the last-level cache)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the hot path runs on a single MI355X and has no multi-GPU "
              f"mode (asked for --gpus {args.gpus}).", file=sys.stderr)
        return 2

    import torch

    import aoship
    import workloads as W

    aoship.init(0)
    log(f"device: {aoship.device_name()}")
    if args.probe:
        return probe(aoship, W, torch, args.layers)
    if args.probe_prefill:
        return probe_prefill(aoship, W, torch)
    if args.probe_model:
        print(json.dumps(model_decode(aoship, W, torch, args.model_layers, 512, 40, 5)), flush=True)
        return 0

    # ---- headline: 7B-shaped decode, one token ----
    T = 1
    dec = MlpCase(aoship, W, 2, T, torch, args.layers)
    dec.combined = False  # route, then the layer: two calls
    ms_two = time_steps(dec, args.steps, args.warmup, torch)
    kt_two = kernel_times(dec, max(20, args.steps // 4), torch)
    dec.combined = FUSED  # the headline: one call, the router inside the gate/up launch
    ms = time_steps(dec, args.steps, args.warmup, torch)
    U = dec.distinct_adapters(aoship)
    kt = kernel_times(dec, max(20, args.steps // 4), torch)
    cfg = dec.cfg
    layer_bytes = W.algorithmic_bytes(cfg, T, U)
    one_launch = "decode_mlp" in kt  # 1-2 tokens: the whole MLP is one launch
    if "mlp1" in kt:  # one token: the whole layer (and the router) in one launch, down matrix in LDS
        gu_ms = kt["mlp1"]
        gu_bytes = layer_bytes + (cfg.n_adapters + T) * cfg.hidden * 4 * dec.combined
        rl_kernel = (("route+" if dec.combined else "") + "mlp1 (one launch: " +
                     ("the router in the first waves, " if dec.combined else "") +
                     "the LoRA x shrink, the int4 gate+up GEMV with the LoRA expand and SwiGLU, the down "
                     "shrink, and the int4 down GEMV from LDS with its expand)")
    elif one_launch:
        gu_ms = kt["decode_mlp"]
        gu_bytes = layer_bytes
        rl_kernel = ("decode_mlp (one launch: the LoRA x shrink and adapter plan, the int4 gate+up GEMV with "
                     "the LoRA expand, SwiGLU and the down shrink's partials, their sum, then the int4 down "
                     "GEMV with its expand)")
    else:
        gu_ms = kt["q4_gemv_gate_up"]
        # with the router in the launch: its weights and the token's features as well
        gu_bytes = gate_up_bytes(cfg, T, U) + (cfg.n_adapters + T) * cfg.hidden * 4 * dec.combined
        rl_kernel = ("route+lora_shrink_x+q4_gemv_gate_up (one launch: the router's workgroups, the adapter plan "
                     "and the LoRA x shrink in its first workgroups, then the int4 gate+up GEMV with the LoRA "
                     "expand and SwiGLU)" if dec.combined else
                     "lora_shrink_x+q4_gemv_gate_up (one launch: the LoRA x shrink in its first workgroups, "
                     "then the int4 gate+up GEMV with the LoRA expand and SwiGLU)")
    achieved = gu_bytes / (gu_ms * 1e-3) / 1e9
    kl = launch_names(kt, dec.combined)
    log(f"decode T=1: {ms * 1e3:.1f} us/step, launches (us): " +
        ", ".join(f"{k} {v * 1e3:.1f}" for k, v in kl.items()))
    result = {
        "metric": METRIC,
        "value": T / (ms * 1e-3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "Qwen2.5-7B-shaped int4 (g64) SwiGLU MLP, 16 rank-16 LoRA adapters on gate/up/down, "
                        "K=4 Q15 router over 3584-dim features, decode of 1 token; each step routes the token "
                        "and runs the next of %d distinct layer copies, both in one aoship_route_mlp_forward "
                        "call" % args.layers,
            "hidden": cfg.hidden, "intermediate": cfg.inter, "tokens": T, "adapters": cfg.n_adapters,
            "rank": cfg.rank, "k": cfg.k, "layers_cycled": args.layers,
        },
        "layer_hbm_gbps": layer_bytes / (ms * 1e-3) / 1e9,
        "roofline": {
            "bound": "hbm",
            "kernel": rl_kernel,
            "achieved": achieved,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBPS,
            "traffic": measured_traffic(MLP1_TRAFFIC_FILE if "mlp1" in kt else TRAFFIC_FILE),
            "algorithmic_bytes": gu_bytes,
            "avg_launch_us": gu_ms * 1e3,
        },
        "kernels_us": {k: v * 1e3 for k, v in kl.items()},
        "decode_t1_two_calls": {"ms_per_step": ms_two, "tok_s": T / (ms_two * 1e-3),
                                "kernels_us": {k: v * 1e3 for k, v in launch_names(kt_two).items()},
                                "note": "the router's launch, then aoship_mlp_forward"},
    }
    log(f"decode T=1 as two calls (route, then aoship_mlp_forward): {ms_two * 1e3:.1f} us/step")
    # the step's bytes, with the router's fp32 weights and features when it routes in the call
    step_bytes = layer_bytes + (cfg.n_adapters + T) * cfg.hidden * 4 * int(bool(dec.combined))
    del dec
    hp = hbm_stream_probe(gate_up_bytes(cfg, T, U), layer_bytes - gate_up_bytes(cfg, T, U), step_bytes)
    if hp:
        result["decode_hbm_probe"] = hp
        log("HBM stream probe: ceiling %.2f TB/s; one launch of %.1f MB %.1f us (%.2f TB/s), %.1f MB %.1f us "
            "(%.2f TB/s); at the decode grids %.1f / %.1f us" % (
                hp["ceiling"]["tbps"], hp["gate_up_bytes"]["bytes"] / 1e6, hp["gate_up_bytes"]["us"],
                hp["gate_up_bytes"]["tbps"], hp["down_bytes"]["bytes"] / 1e6, hp["down_bytes"]["us"],
                hp["down_bytes"]["tbps"], hp["gate_up_bytes_at_592_workgroups"]["us"],
                hp["down_bytes_at_448_workgroups"]["us"]))
        log("HBM stream probe: the one-token launch's %.1f MB in one launch %.1f us" % (
            hp["layer_bytes"]["bytes"] / 1e6, hp["layer_bytes"]["us"]))

    # ---- 8-token decode batch ----
    T8 = 8
    d8 = MlpCase(aoship, W, 2, T8, torch, args.layers)
    d8.combined = False
    ms8_two = time_steps(d8, args.steps, args.warmup, torch)
    d8.combined = FUSED  # routing and the MLP in one aoship_route_mlp_forward call, as the headline
    ms8 = time_steps(d8, args.steps, args.warmup, torch)
    kt8 = kernel_times(d8, max(20, args.steps // 4), torch)
    U8 = d8.distinct_adapters(aoship)
    result["decode_t8"] = {
        "tok_s": T8 / (ms8 * 1e-3),
        "ms_per_step": ms8,
        "distinct_adapters": U8,
        "layer_hbm_gbps": W.algorithmic_bytes(cfg, T8, U8) / (ms8 * 1e-3) / 1e9,
        "kernels_us": {k: v * 1e3 for k, v in launch_names(kt8, d8.combined).items()},
        "two_calls_ms_per_step": ms8_two,
        "note": "one aoship_route_mlp_forward call per step; two_calls_ms_per_step: the router's launch, "
                "then aoship_mlp_forward",
    }
    log(f"decode T=8: {ms8 * 1e3:.1f} us/step (two calls {ms8_two * 1e3:.1f})")
    del d8

    # ---- 2048-token prefill ----
    if not args.skip_prefill:
        pf = MlpCase(aoship, W, 3, 2048, torch, 1)
        # a prefill step is a ~1 ms burst of matrix-core work: the first tens of steps on a GPU that
        # has been running the decode lines run ~6% slower (measured: 969 against 912 us per step,
        # every later window 910-913), so the warm-up covers that before the timed steps
        msp = time_steps(pf, max(5, args.steps // 10), 25, torch)
        kp = kernel_times(pf, max(5, args.steps // 20), torch)
        flops = W.algorithmic_flops(pf.cfg, 2048)
        peak_meas = measured_mfma_peak()
        tflops = flops / (msp * 1e-3) / 1e12
        H, I = pf.cfg.hidden, pf.cfg.inter
        gu_flops = 2 * 2048 * H * 2 * I
        result["prefill"] = {
            "tokens": 2048,
            "tok_s": 2048 / (msp * 1e-3),
            "ms_per_step": msp,
            "algorithmic_tflop": flops / 1e12,
            "achieved_tflops": tflops,
            "mfma_util": tflops / BF16_PEAK_TFLOPS,
            "peak_tflops": BF16_PEAK_TFLOPS,
            "peak_measured_tflops": peak_meas,
            "mfma_util_of_measured_peak": tflops / peak_meas if peak_meas else None,
            "kernels_us": {k: v * 1e3 for k, v in kp.items()},
            "gemm_gate_up_tflops": gu_flops / (kp["q4_gemm_gate_up"] * 1e-3) / 1e12 if "q4_gemm_gate_up" in kp else None,
            "library_bf16_gemm": library_gemm_reference(torch, 2048, H, I),
        }
        # what the step holds besides the layer's launches: the router's launch, and the rest
        # (launch gaps, host-side planning)
        route_ms = time_steps(RouteOnly(pf), 20, 3, torch)
        result["prefill"]["route_us"] = route_ms * 1e3
        result["prefill"]["step_minus_route_and_launches_us"] = (msp - route_ms - sum(kp.values())) * 1e3
        log(f"prefill T=2048: {msp:.3f} ms/step, {tflops:.1f} TFLOP/s; route {route_ms * 1e3:.1f} us; kernels (us): " +
            ", ".join(f"{k} {v * 1e3:.1f}" for k, v in kp.items()))
        del pf

    # ---- C4: attention projections of a 3B-shaped layer for 32 concurrent decode streams ----
    if not args.skip_c4:
        c4 = ProjCase(aoship, W, 4, 32, torch, 24)
        c4.route = False  # the projections alone (rings of the first routing): the roofline figure
        ms_p = time_steps(c4, args.steps, args.warmup, torch)
        kt4 = kernel_times(c4, max(20, args.steps // 4), torch)
        c4.route = True
        ms_s = time_steps(c4, args.steps, args.warmup, torch)
        U4 = c4.distinct_adapters(aoship)
        b4 = c4_bytes(c4.cfg, 32, U4)
        ach = b4 / (ms_p * 1e-3) / 1e9
        result["c4_projections"] = {
            "workload": "Llama-3.2-3B-shaped q/k/v/o projections (3072 -> 3072/1024/1024, o 3072 -> 3072), int4 g64, "
                        "32 rank-16 adapters on all four, 32 decode streams each routed to its own K=4 set from its "
                        "features; 24 distinct layer copies cycled",
            "streams": 32, "distinct_adapters": U4,
            "ms_per_step": ms_s, "tok_s": 32 / (ms_s * 1e-3),
            "projections_ms": ms_p,
            "kernels_us": {k: v * 1e3 for k, v in kt4.items()},
            "roofline": {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": ach / HBM_PEAK_GBPS, "algorithmic_bytes": b4,
                         "note": "q/k/v launch + o launch per step (rings given), bytes = int4 base with scales and "
                                 "biases + the U distinct adapters' bf16 LoRA rows + bf16 activations"},
        }
        log(f"C4 projections, 32 streams: {ms_p * 1e3:.1f} us (projections), {ms_s * 1e3:.1f} us with routing; "
            f"{ach:.0f} GB/s; launches (us): " + ", ".join(f"{k} {v * 1e3:.1f}" for k, v in kt4.items()))
        del c4

    # ---- C5: 32B-shaped MLP, 4096-token prefill, 64 rank-64 adapters, K=8, adversarial routing ----
    if not args.skip_c5:
        c5 = MlpCase(aoship, W, 5, 4096, torch, 1)
        ms5 = time_steps(c5, max(3, args.steps // 40), 4, torch)
        kt5 = kernel_times(c5, 3, torch)
        f5 = W.algorithmic_flops(c5.cfg, 4096)
        tf5 = f5 / (ms5 * 1e-3) / 1e12
        result["c5_stress"] = {
            "workload": "Qwen2.5-32B-shaped int4 (g64) SwiGLU MLP (5120 / 27648), 64 rank-64 adapters, K=8, "
                        "adversarial priors (exact ties, gates rounding to 0 or 1 in Q15), prefill of 4096 tokens",
            "tokens": 4096, "ms_per_step": ms5, "tok_s": 4096 / (ms5 * 1e-3),
            "kernels_us": {k: v * 1e3 for k, v in kt5.items()},
            "roofline": {"bound": "mfma", "achieved": tf5, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": tf5 / BF16_PEAK_TFLOPS, "algorithmic_flop": f5,
                         "note": "route + MLP per step; FLOP = base GEMMs + the K active adapters' shrink and expand"},
        }
        log(f"C5 stress prefill T=4096: {ms5:.3f} ms/step, {tf5:.1f} TFLOP/s; kernels (us): " +
            ", ".join(f"{k} {v * 1e3:.1f}" for k, v in kt5.items()))
        del c5

    # ---- the whole decoder, token by token ----
    if not args.skip_model:
        md = model_decode(aoship, W, torch, args.model_layers, 512, max(20, args.steps // 8), 5)
        result["model_decode"] = md
        log(f"model decode ({md['layers']} layers, context {md['context']}): {md['ms_per_token']:.3f} ms/token, "
            f"{md['tok_s']:.1f} tok/s, ~{md['approx_hbm_gbps']:.0f} GB/s")

    if not args.skip_cpu:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(W)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
