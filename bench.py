"""Benchmark of the FADE tiered-KV hot path on one MI355X.

One step = one fused tiered decode-attention call (one query token per
(batch row, query head)) over the whole synthetic cache of BASELINE
config 1: Llama-3-8B-shaped layer, batch 16, 32 query / 8 KV heads,
head_dim 128, 8192 cached tokens = 4 fp16 sinks + 8124 INT4 middle tokens
(per-channel K / per-token V scales, the reference format) + 64 fp16 recent.

The timed loop rotates over several cache instances (>= 512 MB together)
so the 256 MB Infinity Cache cannot hold the working set; inputs are
resident in HBM before timing starts.  Prints one JSON line.

  python bench.py [--gpus 1] [--steps 200] [--warmup 20]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from fade_amd import _lib  # noqa: E402
from fade_amd import quant as fq  # noqa: E402
from fade_amd import rotated_quant as frq  # noqa: E402
from fade_amd.kernels.tiered_attn import MiddleTier, TieredDecodePlan  # noqa: E402
from fade_amd.synthetic import CONFIGS, kv_tensors  # noqa: E402

HBM_PEAK_GBPS = 8000.0
METRIC = "fused INT4 tiered decode attn latency (µs) + achieved HBM GB/s vs peak, 1 GPU"
N_INSTANCES = 4


def decode_bytes(cfg, fmt: str) -> int:
    """Algorithmic bytes of one decode call: each KV byte once, plus q in and out."""
    D, ns_nr, mid = cfg.D, cfg.n_sink + cfg.recent, cfg.mid
    per_head = ns_nr * D * 4
    if fmt == "int4":
        per_head += mid * D + 2 * D + 2 * mid
    elif fmt == "k4v2":  # reference literal: int8 V codes, S padded to 64, [G, D] fp16 scales
        pad = -(-mid // 64) * 64
        per_head += mid * D // 2 + 2 * D + pad * D + (pad // 64) * D * 2
    elif fmt == "rot2":  # rotated K2/V2: 2-bit packed codes, K per-channel + V per-token scales
        per_head += mid * D // 4 * 2 + 2 * D + 2 * mid
    elif fmt.startswith("asym"):  # asym group-32 "asymKV": codes + fp16 scale and zero per token and group
        kb, vb = int(fmt[4]), int(fmt[5])
        per_head += mid * (D * kb // 8 + D * vb // 8 + 2 * (D // 32) * 2 * 2)
    elif fmt == "fp16":
        per_head += mid * D * 4
    return cfg.B * cfg.Hkv * per_head + 2 * cfg.B * cfg.Hq * D * 2


def build_instances(cfg, fmt: str, dev, seed: int, n: int, dtype=torch.float16):
    """Quantize the middle tier once on the GPU, then clone it into n distinct allocations.
    ``dtype``: the cache's (and model's) float type, float16 or bfloat16."""
    q, k, v = kv_tensors(cfg.B, cfg.Hkv, cfg.S, cfg.D, seed=seed, Hq=cfg.Hq)
    qd, kd, vd = q.to(dev, dtype), k.to(dev, dtype), v.to(dev, dtype)
    del k, v
    ns, nr, S = cfg.n_sink, cfg.recent, cfg.S
    km, vm = kd[:, :, ns : S - nr].contiguous(), vd[:, :, ns : S - nr].contiguous()
    sink = (kd[:, :, :ns].contiguous(), vd[:, :, :ns].contiguous())
    rec = (kd[:, :, S - nr :].contiguous(), vd[:, :, S - nr :].contiguous())
    rot = None
    if fmt == "int4":
        kq, ks = fq.quant_k_int4(km)
        vq, vs = fq.quant_v_int4(vm)
        mid = MiddleTier("int4", kq, vq, ks, vs)
    elif fmt == "k4v2":
        kq, ks = fq.quant_k_int4(km)
        vq, vs = fq.quant_int2_padded(vm, 64)
        mid = MiddleTier("k4v2", kq, vq, ks, vs, group=64, length=cfg.mid)
    elif fmt == "rot2":
        R = torch.from_numpy(np.load(os.path.join(ROOT, "tests", "golden", "rotation_d128_seed42.npy"))).to(dev)
        kq, ks = frq.rotated_quant_k(km, R, 2)
        vq, vs = frq.rotated_quant_v(vm, R, 2)
        mid = MiddleTier("sym", kq, vq, ks, vs, k_bits=2, v_bits=2)
        rot = R  # q, sink and recent stay in the model's basis: the kernel rotates
    elif fmt.startswith("asym"):
        kb, vb = int(fmt[4]), int(fmt[5])
        kq, ks, kz = fq.quant_asym(km, kb, 32)
        vq, vs, vz = fq.quant_asym(vm, vb, 32)
        mid = MiddleTier("asym", kq, vq, ks, vs, kz, vz, k_bits=kb, v_bits=vb, group=32)
    else:
        mid = MiddleTier("fp16", km, vm)
    del kd, vd
    plans = []
    for _ in range(n):
        m = MiddleTier(mid.fmt, *(t.clone() if t is not None else None for t in
                                  (mid.k_codes, mid.v_codes, mid.k_scale, mid.v_scale, mid.k_zero, mid.v_zero)),
                       k_bits=mid.k_bits, v_bits=mid.v_bits, group=mid.group, length=mid.length)
        s = tuple(t.clone() for t in sink)
        r = tuple(t.clone() for t in rec)
        plans.append(TieredDecodePlan(qd, s, m, r, rotation=rot))
    return plans


def time_plans(plans, steps: int, warmup: int, stream):
    """Back-to-back launches rotating over instances; per-call HIP events on the launch stream."""
    for i in range(warmup):
        plans[i % len(plans)].run(stream.cuda_stream)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        for i in range(steps):
            ev[i][0].record(stream)
            plans[i % len(plans)].run(stream.cuda_stream)
            ev[i][1].record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    per_call = np.array([a.elapsed_time(b) for a, b in ev])  # ms
    span_ms = ev[0][0].elapsed_time(ev[-1][1])
    return wall_ms / steps, float(np.median(per_call)), float(per_call.mean()), span_ms / steps


def time_plans_graph(plans, calls: int, replays: int, warmup: int, stream):
    """Decode calls as a serving loop issues them: the instances' calls captured in HIP
    graphs of ``calls`` back-to-back launches (several graphs when ``calls`` is shorter than
    the instance rotation, replayed in turn so that consecutive calls still use different
    instances), each replay bracketed by HIP events on the launch stream.  Returns per-call
    ms (mean, median over the ``replays`` samples) and the wall ms per call of the timed
    region (synchronized on both sides)."""
    for i in range(warmup):
        plans[i % len(plans)].run(stream.cuda_stream)
    torch.cuda.synchronize()
    n_graphs = max(1, len(plans) // calls) if calls < len(plans) else 1
    graphs = []
    for j in range(n_graphs):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(calls):
                plans[(j * calls + i) % len(plans)].run(stream.cuda_stream)
        graphs.append(g)
    with torch.cuda.stream(stream):
        for g in graphs:
            g.replay()  # first replay uploads the graph
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(replays)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        for r, (a, b) in enumerate(ev):
            a.record(stream)
            graphs[r % n_graphs].replay()
            b.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    per_call = np.array([a.elapsed_time(b) for a, b in ev]) / calls
    del graphs
    return float(per_call.mean()), float(np.median(per_call)), wall_ms / (calls * replays)


def graph_split(steps: int, most: int = 32, rotate: int = N_INSTANCES) -> tuple[int, int]:
    """(calls per graph, replays) with calls * replays == steps, calls <= most; a multiple
    of ``rotate`` when one divides steps (no instance runs twice in a row across replays).
    Long graphs keep the replay-launch overhead out of the per-call time; the median over
    many replays comes from a separate statistics pass (``STATS_REPLAYS``)."""
    divs = [d for d in range(1, min(most, steps) + 1) if steps % d == 0]
    rot = [d for d in divs if d % rotate == 0]
    calls = max(rot) if rot else max(divs)
    return calls, steps // calls


STATS_CALLS, STATS_REPLAYS = 20, 10


def settle(plans, stream, ms: float = 200.0) -> int:
    """Untimed decode calls for ``ms`` of wall time before any measurement: the GPU's clocks
    ramp up over the first ~20 ms of work after idle (per-call times fall by ~8% over the
    first few hundred calls).  Returns the number of calls made."""
    n, t0 = 0, time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(20):
            plans[n % len(plans)].run(stream.cuda_stream)
            n += 1
        torch.cuda.synchronize()
    return n


STREAM_WGS = 4096


def stream_read_peak(dev, nbytes: int, stream, calls: int = 20, replays: int = 10) -> dict:
    """Read-only HBM ceiling at the decode's size: ``nbytes`` streamed by one launch of the
    16-byte non-temporal read kernel of libfade_bench.so, rotating over 4 buffers like the
    decode instances, timed over HIP-graph replays like the headline."""
    lib = ctypes.CDLL(os.path.join(ROOT, "fade_amd", "libfade_bench.so"))
    fn = lib.fade_bench_stream_read
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]
    nb = nbytes // 16 * 16
    bufs = [torch.empty(nb, dtype=torch.uint8, device=dev).fill_(i + 1) for i in range(N_INSTANCES)]
    sink = torch.zeros(STREAM_WGS, dtype=torch.int32, device=dev)

    class _P:
        def __init__(self, b):
            self.b = b

        def run(self, s):
            if fn(self.b.data_ptr(), nb, STREAM_WGS, sink.data_ptr(), s) != 0:
                raise RuntimeError("fade_bench_stream_read failed")

    plans = [_P(b) for b in bufs]
    settle(plans, stream, 50.0)
    mean, med, _ = time_plans_graph(plans, calls, replays, 10, stream)
    del bufs
    return {"bytes": nb, "us": round(med * 1e3, 2), "GBps": round(nb / (med * 1e-3) / 1e9, 1),
            "frac_of_8TBps": round(nb / (med * 1e-3) / 1e9 / HBM_PEAK_GBPS, 3),
            "kernel": f"16-byte non-temporal loads, {STREAM_WGS} workgroups of 256 threads, 8 loads in flight each"}


MFMA_F16_PEAK_TFLOPS = 2500.0


class CallPlan:
    """One C-ABI call with preallocated arguments; ``run(stream)`` enqueues it."""

    def __init__(self, name: str, args_fn, keep):
        self.fn = getattr(_lib.load(), name)
        self.name, self.args_fn, self._keep = name, args_fn, keep

    def run(self, stream: int | None = None) -> None:
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        _lib.check(self.fn(*self.args_fn(s)), self.name)


def quant_cases(dev):
    """Middle-tier quantizers at full size: config 1 (reference INT4 K and V),
    config 2 (asymmetric group-32 K4 / V2) and config 2's rotated 2-bit K / V
    (fused rotation + quantize).  Bytes: fp16 read once + codes and scales
    written (a two-phase kernel's re-read of K is not counted)."""
    out = []
    c1 = CONFIGS[1]
    _, k, v = kv_tensors(c1.B, c1.Hkv, c1.S, c1.D, seed=1001, Hq=c1.Hq)
    km = k[:, :, c1.n_sink : c1.S - c1.recent].contiguous().to(dev)
    vm = v[:, :, c1.n_sink : c1.S - c1.recent].contiguous().to(dev)
    del k, v
    B, H, S, D = km.shape
    kp = torch.empty(B, H, S, D // 2, dtype=torch.uint8, device=dev)
    ks = torch.empty(B, H, 1, D, dtype=torch.float16, device=dev)
    nb = ctypes.c_int64(0)
    _lib.check(_lib.load().fade_quant_k_int4_workspace_bytes(B, H, S, D, nb), "ws")
    ws = _lib.workspace(nb.value, dev)
    st = (km.stride(0), km.stride(1), km.stride(2))
    # every lambda binds its arguments as defaults: later cases rebind these names
    out.append(("c1_quant_k_int4", CallPlan("fade_quant_k_int4", lambda s_, km=km, kp=kp, ks=ks, ws=ws, st=st, sh=(B, H, S, D): (
        km.data_ptr(), *sh, *st, kp.data_ptr(), ks.data_ptr(), ws.data_ptr(), ws.numel(), s_),
        (km, kp, ks, ws)), km.numel() * 2 + kp.numel() + ks.numel() * 2))
    vp = torch.empty(B, H, S, D // 2, dtype=torch.uint8, device=dev)
    vs = torch.empty(B, H, S, 1, dtype=torch.float16, device=dev)
    out.append(("c1_quant_v_int4", CallPlan("fade_quant_v_int4", lambda s_, vm=vm, vp=vp, vs=vs, st=st, sh=(B, H, S, D): (
        vm.data_ptr(), *sh, *st, vp.data_ptr(), vs.data_ptr(), s_), (vm, vp, vs)),
        vm.numel() * 2 + vp.numel() + vs.numel() * 2))
    # dequant_int4 of the two tiers above back to fp16 (materialize's middle tier):
    # K with its per-channel scale, V with its per-token scale
    for name, pk, sc, axis in (("c1_dequant_int4_k", kp, ks, _lib.AXIS_CHANNEL), ("c1_dequant_int4_v", vp, vs, _lib.AXIS_TOKEN)):
        dq = torch.empty(B, H, S, D, dtype=torch.float16, device=dev)
        out.append((name, CallPlan("fade_dequant_sym", lambda s_, pk=pk, sc=sc, dq=dq, axis=axis, sh=(B, H, S, D): (
            pk.data_ptr(), sc.data_ptr(), 4, axis, *sh, dq.data_ptr(), s_), (pk, sc, dq)),
            pk.numel() + sc.numel() * 2 + dq.numel() * 2))
    c2 = CONFIGS[2]
    _, k2, v2 = kv_tensors(c2.B, c2.Hkv, c2.S, c2.D, seed=1002, Hq=c2.Hq)
    for name, x, bits in (("c2_quant_asym_k4", k2, 4), ("c2_quant_asym_v2", v2, 2)):
        xm = x[:, :, c2.n_sink : c2.S - c2.recent].contiguous().to(dev)
        B, H, S, D = xm.shape
        pk = torch.empty(B, H, S, D * bits // 8, dtype=torch.uint8, device=dev)
        sc = torch.empty(B, H, S, D // 32, dtype=torch.float16, device=dev)
        zp = torch.empty_like(sc)
        xs = (xm.stride(0), xm.stride(1), xm.stride(2))
        out.append((name, CallPlan("fade_quant_asym", lambda s_, xm=xm, pk=pk, sc=sc, zp=zp, xs=xs, bits=bits, sh=(B, H, S, D): (
            xm.data_ptr(), *sh, *xs, bits, 32, pk.data_ptr(), sc.data_ptr(), zp.data_ptr(), s_), (xm, pk, sc, zp)),
            xm.numel() * 2 + pk.numel() + 2 * sc.numel() * 2))
    # config 2's V in the reference's literal grouped INT2 (the K4 + V2 format's V, the INT2
    # tier): int8 codes and a per-(64-token group, channel) fp16 scale
    xm = v2[:, :, c2.n_sink : c2.S - c2.recent].contiguous().to(dev)
    B, H, S, D = xm.shape
    S_pad = -(-S // 64) * 64
    cq = torch.empty(B, H, S_pad, D, dtype=torch.int8, device=dev)
    cs = torch.empty(B, H, S_pad // 64, D, dtype=torch.float16, device=dev)
    xs = (xm.stride(0), xm.stride(1), xm.stride(2))
    out.append(("c2_quant_int2_grouped_v", CallPlan("fade_quant_int2_grouped", lambda s_, xm=xm, cq=cq, cs=cs, xs=xs, sh=(B, H, S, S_pad, D): (
        xm.data_ptr(), *sh, *xs, 64, cq.data_ptr(), cs.data_ptr(), s_), (xm, cq, cs)),
        xm.numel() * 2 + cq.numel() + cs.numel() * 2))
    # and back to fp16 (the INT2 tier's fp16 copy for the fused attention): reads the
    # codes the line above wrote
    dq = torch.empty_like(xm)
    out.append(("c2_dequant_int2_grouped_v", CallPlan("fade_dequant_int2_grouped", lambda s_, cq=cq, cs=cs, dq=dq, sh=(B, H, S_pad, D), S_=S: (
        cq.data_ptr(), cs.data_ptr(), *sh, 64, S_, dq.data_ptr(), s_), (cq, cs, dq)),
        cq.numel() + cs.numel() * 2 + dq.numel() * 2))
    # rotated backend at config 2's 2-bit middle tier: fused MFMA rotation + quantize
    R = torch.from_numpy(np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests", "golden",
                                              "rotation_d128_seed42.npy"))).to(dev)
    for name, x, axis in (("c2_rotate_quant_k2", k2, _lib.AXIS_CHANNEL), ("c2_rotate_quant_v2", v2, _lib.AXIS_TOKEN)):
        xm = x[:, :, c2.n_sink : c2.S - c2.recent].contiguous().to(dev)
        B, H, S, D = xm.shape
        pk = torch.empty(B, H, S, D // 4, dtype=torch.uint8, device=dev)
        sc = torch.empty(B * H * (S if axis == _lib.AXIS_TOKEN else D), dtype=torch.float16, device=dev)
        nb = ctypes.c_int64(0)
        _lib.check(_lib.load().fade_rotate_quant_workspace_bytes(B, H, S, D, axis, nb), "ws")
        ws = _lib.workspace(nb.value, dev)
        xs = (xm.stride(0), xm.stride(1), xm.stride(2))
        out.append((name, CallPlan("fade_rotate_quant", lambda s_, xm=xm, pk=pk, sc=sc, ws=ws, xs=xs, axis=axis, sh=(B, H, S, D), R=R: (
            xm.data_ptr(), *sh, *xs, R.data_ptr(), 2, axis, pk.data_ptr(), sc.data_ptr(), ws.data_ptr(), ws.numel(), s_),
            (xm, pk, sc, ws, R)), xm.numel() * 2 + pk.numel() + sc.numel() * 2))
    return out


def rerope_case(dev):
    """Config 3: eviction re-RoPE of the kept rows (K un-RoPE at the old
    positions, re-RoPE at 0..n_kept-1) plus the V gather, B=8, Hkv=4, S=4096,
    kept = 4 sink + 400 highest-scoring middle + 64 recent rows."""
    from fade_amd.rope import Vanilla
    from fade_amd.synthetic import exp_scores

    B, H, S, D = 8, 4, 4096, 128
    _, k, v = kv_tensors(B, H, S, D, seed=1003, Hq=28)
    rope = Vanilla(theta=1.0e6, head_dim=D)
    cos_o, sin_o = rope.host_cos_sin(torch.arange(S))
    kf = k.float()
    half = D // 2
    rot = torch.cat((-kf[..., half:], kf[..., :half]), dim=-1)
    k_post = (kf * cos_o + rot * sin_o).half()  # K after RoPE at positions 0..S-1
    sc = exp_scores(S, 1003)
    mid = torch.arange(4, S - 64)
    top = mid[torch.argsort(sc[4 : S - 64], descending=True)[:400]]
    keep = torch.sort(torch.cat((torch.arange(4), top, torch.arange(S - 64, S)))).values
    n = int(keep.numel())
    cos_n, sin_n = rope.host_cos_sin(torch.arange(n))
    kd, vd, kp = k_post.to(dev), v.to(dev), keep.to(dev)
    tabs = [t.contiguous().to(dev) for t in (cos_o, sin_o, cos_n, sin_n)]
    ko = torch.empty(B, H, n, D, dtype=torch.float16, device=dev)
    vo = torch.empty_like(ko)
    plan = CallPlan("fade_rerope_gather", lambda s_: (
        kd.data_ptr(), *kd.stride()[:3], vd.data_ptr(), *vd.stride()[:3], B, H, S, D, kp.data_ptr(), n,
        *(t.data_ptr() for t in tabs), ko.data_ptr(), vo.data_ptr(), s_), (kd, vd, kp, tabs, ko, vo))
    return plan, 4 * B * H * n * D * 2, n


def reassign_case(dev, n_inst: int = 8):
    """Config 3 tier reassignment of one layer, wall-clock per call (host work and
    syncs included), device path vs the host path (the reference's op sequence):
    B=8, Hkv=4; a cache of 4 sink + 3964 INT4 + 128 fp16 recent tokens (4096)
    keeps 4 sink + the 400 best-scoring middle + 64 recent (eviction, re-RoPE,
    middle requantized)."""
    from fade_amd.cache import TieredKVCache
    from fade_amd.policy import _assign_one_layer
    from fade_amd.synthetic import exp_scores

    B, H, D = 8, 4, 128
    _, k, v = kv_tensors(B, H, 4096, D, seed=1003, Hq=28)
    kd, vd = k.to(dev), v.to(dev)
    tiers0 = _assign_one_layer(4032, torch.zeros(4032), 4, 64, None, 0)
    tiers = _assign_one_layer(4096, exp_scores(4096, 1003), 4, 64, 400, 0)
    out = {}
    for name, device_path in (("device", True), ("host", False)):
        caches = []
        for _ in range(n_inst):
            c = TieredKVCache(n_sink=4, recent_window=64, int4_budget=400, int2_budget=0, head_dim=D)
            c.device_reassign = device_path
            c.update(kd[:, :, :4032], vd[:, :, :4032], 0)
            c.apply_tier_assignment(0, tiers0)
            c.update(kd[:, :, 4032:], vd[:, :, 4032:], 0)
            caches.append(c)
        caches[0].apply_tier_assignment(0, tiers)  # warm-up (RoPE table, allocator)
        torch.cuda.synchronize()
        times = []
        for c in caches[1:]:
            t0 = time.perf_counter()
            c.apply_tier_assignment(0, tiers)
            torch.cuda.synchronize()
            times.append((time.perf_counter() - t0) * 1e6)
        out[name] = round(float(np.median(times)), 1)
        del caches
        torch.cuda.empty_cache()
    return out


def per_sequence_case(dev, n_inst: int = 4):
    """The reference's per-sequence assignment (zero-padded rows) at config 3's cache
    shape, wall-clock per call, device path vs host path (the reference's op
    sequence): B=8 rows of 4096 tokens, Hkv=4, each row keeping 4 sink + its own 400
    best-scoring middle + 128 recent tokens (per-row eviction, re-RoPE, middle quantized)."""
    from fade_amd.cache import TieredKVCache
    from fade_amd.policy import _assign_one_layer
    from fade_amd.synthetic import exp_scores

    B, H, S, D = 8, 4, 4096, 128
    _, k, v = kv_tensors(B, H, S, D, seed=1003, Hq=28)
    kd, vd = k.to(dev), v.to(dev)
    tiers = torch.stack([_assign_one_layer(S, exp_scores(S, 1100 + b), 4, 128, 400, 0) for b in range(B)])
    out = {}
    for name, device_path in (("device", True), ("host", False)):
        times = []
        for i in range(n_inst + 1):
            c = TieredKVCache(n_sink=4, recent_window=128, int4_budget=400, int2_budget=0, head_dim=D)
            c.device_reassign = device_path
            c.update(kd, vd, 0)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            c.apply_tier_assignment_per_sequence(0, tiers)
            torch.cuda.synchronize()
            if i:  # the first call warms up the RoPE table and the allocator
                times.append((time.perf_counter() - t0) * 1e6)
            del c
        out[name] = round(float(np.median(times)), 1)
    torch.cuda.empty_cache()
    return out


def gqa_cfg(B: int = 8, S: int = 4096, Hq: int = 28, Hkv: int = 4):
    """Config 3's model shape (Hq=28, Hkv=4: 7 query heads per kv head), reference INT4
    middle, sink 4, recent 128."""
    return type("Cfg", (), dict(B=B, Hq=Hq, Hkv=Hkv, S=S, D=128, n_sink=4, recent=128, mid=S - 132))


# --pmc-config 3: the GQA-7 decode at B=16, S=8192 (the eight-head one-pass instance)
PMC_CONFIGS = {1: CONFIGS[1], 2: CONFIGS[2], 3: gqa_cfg(16, 8192)}


def gqa7_decode_case(dev, B: int = 8, S: int = 4096, Hq: int = 28, Hkv: int = 4):
    """Decode at config 3's model shape (B=8, S=4096 by default): the INT4 kernel with
    all heads of a kv head in one pass (the default) against the general matrix-core
    kernel (kernel=3)."""
    cfg = gqa_cfg(B, S, Hq, Hkv)
    plans = build_instances(cfg, "int4", dev, 1003, N_INSTANCES)
    general = [TieredDecodePlan(*p._keep[:4], kernel=3) for p in plans]
    return plans, general, decode_bytes(cfg, "int4")


def copy_peak(dev, stream) -> float:
    """Device-to-device copy of 1 GiB (read + write), GB/s: the measured streaming ceiling."""
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    with torch.cuda.stream(stream):
        for _ in range(3):
            dst.copy_(src)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(10):
            dst.copy_(src)
        b.record(stream)
    torch.cuda.synchronize()
    return 2 * (1 << 30) * 10 / (a.elapsed_time(b) * 1e-3) / 1e9


def prefill_case(dev, seed: int = 1004, B: int = 32, Hq: int = 32, Hkv: int = 8, D: int = 128, Lmax: int = 16384):
    """Config 4: 32 rows, cached lengths ~U[512, 16384], 128-token chunk, 32/8 heads, reference INT4
    middle tier (sink 4, recent 64).  Codes, scales and fp16 tiers are random device tensors (the
    kernel's timing does not depend on their values); rows are dispatched longest first.  The
    keyword arguments give other shapes of the same kind (the head_dim-256 line)."""
    from fade_amd.kernels.prefill import TieredPrefillPlan

    Sq, ns, nr = 128, 4, 64
    gen = torch.Generator().manual_seed(seed)
    L = torch.randint(512, Lmax + 1, (B,), generator=gen)
    nm = L - ns - nr
    cap = int(nm.max())
    g = torch.Generator(device=dev).manual_seed(seed)
    rnd = lambda *shape: torch.randn(*shape, generator=g, device=dev).to(torch.float16)  # noqa: E731
    codes = lambda: torch.randint(0, 256, (B, Hkv, cap, D // 2), generator=g, device=dev, dtype=torch.uint8)  # noqa: E731
    from fade_amd.kernels import MiddleTier

    mid = MiddleTier("int4", codes(), codes(), (rnd(B, Hkv, 1, D).abs() * 0.3 + 0.05), (rnd(B, Hkv, cap, 1).abs() * 0.3 + 0.05))
    lens = torch.stack([torch.full((B,), ns), nm, torch.full((B,), nr)], dim=1).to(torch.int32)
    order = torch.argsort(L, descending=True).to(torch.int32)
    plan = TieredPrefillPlan(rnd(B, Hq, Sq, D), (rnd(B, Hkv, Sq, D), rnd(B, Hkv, Sq, D)), (rnd(B, Hkv, ns, D), rnd(B, Hkv, ns, D)),
                             mid, (rnd(B, Hkv, nr, D), rnd(B, Hkv, nr, D)), lens=lens, order=order)
    # useful MACs: every (query head, query j) row against its L_b + j + 1 visible keys, QK^T and PV
    j = torch.arange(Sq, dtype=torch.float64)
    flops = float(sum(Hq * (L[b] + j + 1).sum() * D * 4 for b in range(B)))
    nbytes = int(B * Hkv * (nm.sum() / B * D + 2 * D + 2 * nm.sum() / B + (ns + nr + Sq) * D * 4) + 2 * B * Hq * Sq * D * 2)
    return plan, flops, nbytes


def ragged_decode_case(dev, seed: int = 1004):
    """Config 4's batch decoding one token: 32 rows, L_b ~U[512, 16384], 32/8 heads, reference
    INT4 middle (sink 4, recent 64).  Three layouts of the same tokens: per-row lengths over
    padded tensors, a paged middle tier (64-token pages of one pool), and every row padded to
    the longest (what a zero-padded per-sequence cache reads).  Bytes: each row's own tokens."""
    from fade_amd.kernels import MiddleTier
    from fade_amd.kernels.tiered_attn import paginate_middle

    B, Hq, Hkv, D, ns, nr = 32, 32, 8, 128, 4, 64
    gen = torch.Generator().manual_seed(seed)
    L = torch.randint(512, 16385, (B,), generator=gen)
    nm = L - ns - nr
    cap = int(nm.max())
    g = torch.Generator(device=dev).manual_seed(seed)
    rnd = lambda *shape: torch.randn(*shape, generator=g, device=dev).to(torch.float16)  # noqa: E731
    codes = lambda: torch.randint(0, 256, (B, Hkv, cap, D // 2), generator=g, device=dev, dtype=torch.uint8)  # noqa: E731
    mid = MiddleTier("int4", codes(), codes(), rnd(B, Hkv, 1, D).abs() * 0.3 + 0.05, rnd(B, Hkv, cap, 1).abs() * 0.3 + 0.05)
    sink, rec = (rnd(B, Hkv, ns, D), rnd(B, Hkv, ns, D)), (rnd(B, Hkv, nr, D), rnd(B, Hkv, nr, D))
    q = rnd(B, Hq, 1, D)
    lens = torch.stack([torch.full((B,), ns), nm, torch.full((B,), nr)], dim=1).to(torch.int32).to(dev)
    paged = paginate_middle(mid, nm.tolist())
    plans = {
        "lens": TieredDecodePlan(q, sink, mid, rec, lens=lens),
        "paged": TieredDecodePlan(q, sink, paged, rec, lens=lens),
        "padded_to_max": TieredDecodePlan(q, sink, mid, rec),
    }
    nbytes = int(Hkv * (B * (ns + nr) * D * 4 + int(nm.sum()) * (D + 2) + B * 2 * D) + 2 * B * Hq * D * 2)
    return plans, nbytes, int(paged.k_codes.shape[0])


def cpu_baseline(cfg, plans) -> dict:
    """The reference's CPU decode step (oracle/torch_cpu.py: unpack + dequantize,
    concatenate the tiers, GQA expansion, SDPA) over the whole config-1 batch (all 16
    rows), in both working dtypes of the reference's CPU path: fp16 cache with fp32
    SDPA, and fp32 throughout.  Codes come from the first GPU instance (bit-identical
    to the oracle's quantizer); median of 5 calls after 2 warmups, per mode."""
    from oracle import torch_cpu

    try:
        import psutil

        phys = psutil.cpu_count(logical=False)
    except Exception:  # pragma: no cover
        phys = None
    threads = torch.get_num_threads()
    q, sink, mid, rec = plans[0]._keep[:4]
    host = lambda t: t.detach().to("cpu")  # noqa: E731
    qc = host(q)
    sk = (host(sink[0]), host(sink[1]))
    rc = (host(rec[0]), host(rec[1]))
    md = (host(mid.k_codes), host(mid.k_scale), host(mid.v_codes), host(mid.v_scale))
    out = {}
    for mode in ("fp16", "fp32"):
        times = []
        for i in range(7):
            t0 = time.perf_counter()
            torch_cpu.decode_step(qc, sk, md, rc, mode=mode)
            if i >= 2:
                times.append(time.perf_counter() - t0)
        out[mode] = round(float(np.median(times)) * 1e6, 1)
    return {
        "value": out["fp16"],
        "unit": "us per decode call (config 1, whole batch)",
        "cores": int(threads),
        "kind": "port",
        "sample": f"all {cfg.B} rows of config 1, one decode call = unpack + dequantize + cat + GQA expand + "
        f"SDPA (torch CPU restatement of fade/quant.py:46-58,124-127, fade/cache.py:715-808, "
        f"fade/kernels/int4_attention.py:179-202); median of 5 after 2 warmups per mode; value = fp16 cache "
        f"with fp32 SDPA; fp32 throughout = {out['fp32']} us; {threads} torch threads on a host with "
        f"{phys} physical cores / {os.cpu_count()} logical CPUs",
        "fp32_us": out["fp32"],
        "physical_cores": phys,
    }


COPY_MIB = 256
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_int4_c1_traffic.json")
TRAFFIC_FILE_C2 = os.path.join(ROOT, "profiles", "decode_c2_32k_traffic.json")
TRAFFIC_FILE_GQA = os.path.join(ROOT, "profiles", "decode_gqa7_traffic.json")


def pmc_pass(steps: int, config: int = 1, fmt: str = "int4") -> int:
    """Short run for ``rocprofv3 --pmc``: a plain copy of known size (the counter
    calibration), then ``steps`` decode calls of config ``config`` (1 or 2) in
    middle format ``fmt`` (int4, k4v2, rot2, asym42, ...)."""
    dev = torch.device("cuda:0")
    src = torch.ones(COPY_MIB << 18, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    plans = build_instances(PMC_CONFIGS[config], fmt, dev, 1000 + config, N_INSTANCES)
    for i in range(steps):
        plans[i % len(plans)].run()
    torch.cuda.synchronize()
    print(json.dumps({"pmc_pass": True, "copy_MiB": COPY_MIB, "config": config, "fmt": fmt, "decode_calls": steps}))
    return 0


def prefill_pass(calls: int) -> int:
    """Short run for ``rocprofv3 --pmc`` on the config-4 ragged prefill: ``calls`` launches."""
    dev = torch.device("cuda:0")
    plan, _, _ = prefill_case(dev)
    for _ in range(calls):
        plan.run()
    torch.cuda.synchronize()
    print(json.dumps({"prefill_pass": True, "prefill_calls": calls}))
    return 0


def portable_pass(calls: int, head_dim: int) -> int:
    """``calls`` launches of the portable decode kernel at another head dim (B=16,
    32/8 heads, S=8192, reference INT4 middle), for ``rocprofv3`` runs; prints the
    mean call time (HIP events) of 200 more."""
    dev = torch.device("cuda:0")
    B, Hq, Hkv, S, D, ns, nr = 16, 32, 8, 8192, head_dim, 4, 64
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, Hq, 1, D, device=dev, generator=g).half()
    k = torch.randn(B, Hkv, S, D, device=dev, generator=g).half()
    v = torch.randn(B, Hkv, S, D, device=dev, generator=g).half()
    kq, ks = fq.quant_k_int4(k[:, :, ns:S - nr].contiguous())
    vq, vs = fq.quant_v_int4(v[:, :, ns:S - nr].contiguous())
    plan = TieredDecodePlan(q, (k[:, :, :ns].contiguous(), v[:, :, :ns].contiguous()), MiddleTier("int4", kq, vq, ks, vs),
                            (k[:, :, S - nr:].contiguous(), v[:, :, S - nr:].contiguous()), kernel=1)
    for _ in range(calls):
        plan.run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(200):
        plan.run()
    e1.record()
    torch.cuda.synchronize()
    print(json.dumps({"portable_pass": True, "head_dim": D, "calls": calls + 200,
                      "us_per_call": round(e0.elapsed_time(e1) / 200 * 1e3, 2)}))
    return 0


def summarize_pmc(fetch_dir: str, write_dir: str, config: int = 1, fmt: str = "int4") -> int:
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of the decode kernel, scaled by
    what the same counters read for the copy kernel (which moves COPY_MIB each way).
    Config 1 INT4 goes to TRAFFIC_FILE (the headline line's ``traffic``); config-2
    formats go to one entry each of TRAFFIC_FILE_C2, the GQA-7 shape (config 3) to
    TRAFFIC_FILE_GQA."""
    import csv

    def per_kernel(d: str, counter: str):
        path = None
        for root, _, files in os.walk(d):
            for f in files:
                if f.endswith("counter_collection.csv"):
                    path = os.path.join(root, f)
        if path is None:
            raise SystemExit(f"no counter_collection.csv under {d}")
        rows = []
        with open(path) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] == counter:
                    rows.append((r["Kernel_Name"], float(r["Counter_Value"])))
        return rows

    out = {"unit": "bytes per dispatch", "copy_bytes_each_way": COPY_MIB << 20}
    for counter, d, key in (("FETCH_SIZE", fetch_dir, "fetch"), ("WRITE_SIZE", write_dir, "write")):
        rows = per_kernel(d, counter)
        # the calibration copies are the three largest copy dispatches of the run
        copy = sorted((v for k, v in rows if "copy" in k.lower()), reverse=True)[:3]
        dec = [v for k, v in rows if "decode_packed_kernel" in k]
        if len(copy) < 3 or not dec:
            raise SystemExit(f"{counter}: calibration copy or decode kernel missing in {d}")
        copy_kib = float(np.median(copy))
        factor = (COPY_MIB << 10) / copy_kib
        dec_kib = float(np.mean(dec))
        out[f"{key}_counter_KiB"] = round(dec_kib, 1)
        out[f"{key}_copy_counter_KiB"] = round(copy_kib, 1)
        out[f"{key}_scale"] = round(factor, 4)
        out[f"{key}_bytes"] = int(dec_kib * 1024 * factor)
    out["hbm_bytes_per_call"] = out["fetch_bytes"] + out["write_bytes"]
    out["algorithmic_bytes_per_call"] = decode_bytes(PMC_CONFIGS[config], fmt)
    out["traffic_ratio"] = round(out["hbm_bytes_per_call"] / out["algorithmic_bytes_per_call"], 4)
    os.makedirs(os.path.dirname(TRAFFIC_FILE), exist_ok=True)
    if config == 1 and fmt == "int4":
        with open(TRAFFIC_FILE, "w") as f:
            json.dump(out, f, indent=1)
            f.write("\n")
    else:
        path = TRAFFIC_FILE_C2 if config == 2 else TRAFFIC_FILE_GQA
        allf = {}
        if os.path.exists(path):
            with open(path) as f:
                allf = json.load(f)
        allf[f"c{config}_{fmt}"] = out
        with open(path, "w") as f:
            json.dump(allf, f, indent=1, sort_keys=True)
            f.write("\n")
    print(json.dumps(out))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="only the config-1 INT4 line")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="copy calibration + --steps decode calls, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--prefill-pass", action="store_true",
                    help="--steps config-4 prefill calls only, for rocprofv3 --pmc SQ counters")
    ap.add_argument("--portable-pass", type=int, metavar="HEAD_DIM",
                    help="--steps calls of the portable decode kernel at HEAD_DIM (32, 64, 256), for rocprofv3")
    ap.add_argument("--pmc-config", type=int, default=1, choices=(1, 2, 3),
                    help="config of --pmc-pass / --summarize-pmc (default 1; 3: GQA-7 at B=16, S=8192)")
    ap.add_argument("--pmc-fmt", default="int4", help="middle format of --pmc-pass / --summarize-pmc (default int4)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn two rocprofv3 --pmc output folders into " + os.path.relpath(TRAFFIC_FILE, ROOT))
    args = ap.parse_args()
    if args.summarize_pmc:
        return summarize_pmc(*args.summarize_pmc, config=args.pmc_config, fmt=args.pmc_fmt)
    if args.gpus != 1:
        print(
            "bench.py: this build measures one GPU; the decode path shards by batch / kv head "
            "(no exchange) and is not run across GPUs here.",
            file=sys.stderr,
        )
        return 2
    if args.pmc_pass:
        return pmc_pass(args.steps, args.pmc_config, args.pmc_fmt)
    if args.prefill_pass:
        return prefill_pass(args.steps)
    if args.portable_pass:
        return portable_pass(args.steps, args.portable_pass)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(dev)
    cfg = CONFIGS[1]

    plans = build_instances(cfg, "int4", dev, 1001, N_INSTANCES)
    settled = settle(plans, stream)
    _, eager_med_ms, eager_mean_ms, _ = time_plans(plans, args.steps, args.warmup, stream)
    calls, replays = graph_split(args.steps)
    mean_ms, _, ms_step = time_plans_graph(plans, calls, replays, args.warmup, stream)
    # statistics pass (not the timed K steps): the per-call median over STATS_REPLAYS replays
    _, med_ms, _ = time_plans_graph(plans, STATS_CALLS, STATS_REPLAYS, 0, stream)
    nbytes = decode_bytes(cfg, "int4")
    achieved = nbytes / (mean_ms * 1e-3) / 1e9
    cpu = None if args.no_cpu_baseline else cpu_baseline(cfg, plans)
    del plans
    torch.cuda.empty_cache()
    peak = stream_read_peak(dev, nbytes, stream)
    torch.cuda.empty_cache()

    def graph_us(pl) -> float:
        """Per-call µs of other decode workloads: settled, then the median of 10 replays of
        a 20-call graph rotating over the instances."""
        settle(pl, stream, 50.0)
        return time_plans_graph(pl, 20, 10, 5, stream)[1] * 1e3

    extra = {"stream_read_ceiling_c1_bytes": peak}
    if not args.no_extra:
        fp = build_instances(cfg, "fp16", dev, 1001, N_INSTANCES)
        fus = graph_us(fp)
        fb = decode_bytes(cfg, "fp16")
        extra["c1_fp16_flash_decode"] = {
            "us": round(fus, 2), "GBps": round(fb / (fus * 1e-6) / 1e9, 1), "bytes": fb,
            "int4_speedup": round(fus / (med_ms * 1e3), 2),
        }
        del fp
        torch.cuda.empty_cache()
        # config 1 in the format BASELINE states (asymmetric group-32 INT4 K and V)
        pa = build_instances(cfg, "asym44", dev, 1001, N_INSTANCES)
        amean = graph_us(pa) * 1e-3
        ab = decode_bytes(cfg, "asym44")
        extra["c1_asym_g32_k4v4"] = {
            "us": round(amean * 1e3, 2), "GBps": round(ab / (amean * 1e-3) / 1e9, 1), "bytes": ab,
            "frac_of_peak": round(ab / (amean * 1e-3) / 1e9 / HBM_PEAK_GBPS, 3),
        }
        del pa
        torch.cuda.empty_cache()
        # config 1 on a bfloat16 cache (bf16 models: q, fp16-layout tiers, scales and output
        # in bf16; bf16 MFMAs for P V)
        pb = build_instances(cfg, "int4", dev, 1001, N_INSTANCES, dtype=torch.bfloat16)
        bmean = graph_us(pb) * 1e-3
        extra["c1_bf16_int4"] = {
            "us": round(bmean * 1e3, 2), "GBps": round(nbytes / (bmean * 1e-3) / 1e9, 1), "bytes": nbytes,
            "frac_of_peak": round(nbytes / (bmean * 1e-3) / 1e9 / HBM_PEAK_GBPS, 3),
        }
        del pb
        torch.cuda.empty_cache()
        pf, pflops, pbytes = prefill_case(dev)
        # 40 warmup calls: this MFMA-bound kernel's per-call time keeps falling
        # over its first ~30-50 calls (clock and TLB warm-up); steady state is timed
        _, _, pmean, _ = time_plans([pf], max(10, args.steps // 10), 40, stream)
        extra["c4_prefill_ragged"] = {
            "us": round(pmean * 1e3, 1), "TFLOPs": round(pflops / (pmean * 1e-3) / 1e12, 1),
            "mfma_frac_f16_dense": round(pflops / (pmean * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 3),
            "useful_flops": pflops, "GBps": round(pbytes / (pmean * 1e-3) / 1e9, 1),
        }
        del pf
        # the same kind of ragged chunk prefill at head_dim 256 (Gemma-style 16/8 heads;
        # 16 rows of L ~U[512, 8192]): the capacity-256 instance at one wave per SIMD
        pf, pflops, pbytes = prefill_case(dev, 1005, B=16, Hq=16, Hkv=8, D=256, Lmax=8192)
        _, _, pmean, _ = time_plans([pf], max(10, args.steps // 10), 40, stream)
        extra["c4_prefill_ragged_d256_16_8"] = {
            "us": round(pmean * 1e3, 1), "TFLOPs": round(pflops / (pmean * 1e-3) / 1e12, 1),
            "mfma_frac_f16_dense": round(pflops / (pmean * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 3),
            "useful_flops": pflops,
        }
        del pf
        torch.cuda.empty_cache()
        for name, plan, nbytes_q in quant_cases(dev):
            _, _, qmean, _ = time_plans([plan], max(20, args.steps // 4), 5, stream)
            extra[name] = {"us": round(qmean * 1e3, 2), "GBps": round(nbytes_q / (qmean * 1e-3) / 1e9, 1),
                           "bytes": nbytes_q, "frac_of_peak": round(nbytes_q / (qmean * 1e-3) / 1e9 / HBM_PEAK_GBPS, 3)}
        torch.cuda.empty_cache()
        rp, rbytes, n_kept = rerope_case(dev)
        _, _, rmean, _ = time_plans([rp], max(20, args.steps // 4), 5, stream)
        extra["c3_rerope_gather"] = {"us": round(rmean * 1e3, 2), "GBps": round(rbytes / (rmean * 1e-3) / 1e9, 1),
                                     "bytes": rbytes, "n_kept": n_kept}
        del rp
        rplans, rdb, n_pages = ragged_decode_case(dev)
        rd = {}
        for name, plan in rplans.items():
            _, _, rmean_d, _ = time_plans([plan], max(20, args.steps // 4), 5, stream)
            rd[name] = round(rmean_d * 1e3, 2)
        extra["c4_ragged_decode"] = {"us": rd, "bytes_own_tokens": rdb, "pool_pages": n_pages,
                                     "GBps_lens": round(rdb / (rd["lens"] * 1e-6) / 1e9, 1),
                                     "GBps_paged": round(rdb / (rd["paged"] * 1e-6) / 1e9, 1)}
        del rplans
        torch.cuda.empty_cache()
        ra = reassign_case(dev)
        extra["c3_reassign_layer_wall_us"] = {"device_path": ra["device"], "host_path": ra["host"],
                                              "speedup": round(ra["host"] / ra["device"], 2)}
        ps = per_sequence_case(dev)
        extra["c3_per_sequence_assignment_wall_us"] = {"device_path": ps["device"], "host_path": ps["host"],
                                                       "speedup": round(ps["host"] / ps["device"], 2)}
        g2, gg, gb = gqa7_decode_case(dev)
        g2mean, ggmean = graph_us(g2) * 1e-3, graph_us(gg) * 1e-3
        extra["c3_shape_decode_gqa7_int4"] = {
            "us_int4_kernel": round(g2mean * 1e3, 2), "us_general_kernel": round(ggmean * 1e3, 2),
            "bytes": gb, "GBps_int4_kernel": round(gb / (g2mean * 1e-3) / 1e9, 1),
        }
        del g2, gg
        torch.cuda.empty_cache()
        # the same model shape at a size that is not launch-bound
        g2, gg, gb = gqa7_decode_case(dev, B=16, S=8192)
        g2mean, ggmean = graph_us(g2) * 1e-3, graph_us(gg) * 1e-3
        extra["c3_shape_b16_s8192_decode_gqa7_int4"] = {
            "us_int4_kernel": round(g2mean * 1e3, 2), "us_general_kernel": round(ggmean * 1e3, 2),
            "bytes": gb, "GBps_int4_kernel": round(gb / (g2mean * 1e-3) / 1e9, 1),
            "frac_of_peak": round(gb / (g2mean * 1e-3) / 1e9 / HBM_PEAK_GBPS, 3),
        }
        del g2, gg
        torch.cuda.empty_cache()
        # config 1's shape at head_dim 64: the general matrix-core kernel (the automatic
        # choice at this head_dim) against the portable one (kernel=1)
        c64 = type("Cfg", (), dict(B=16, Hq=32, Hkv=8, S=8192, D=64, n_sink=4, recent=64, mid=8192 - 68))
        m64 = build_instances(c64, "int4", dev, 1006, N_INSTANCES)
        v64 = [TieredDecodePlan(*pl._keep[:4], kernel=1) for pl in m64]
        mmean, vmean = graph_us(m64) * 1e-3, graph_us(v64) * 1e-3
        b64 = decode_bytes(c64, "int4")
        extra["c1_shape_d64_decode_int4"] = {
            "us": round(mmean * 1e3, 2), "us_portable_kernel": round(vmean * 1e3, 2), "bytes": b64,
            "GBps": round(b64 / (mmean * 1e-3) / 1e9, 1),
            "frac_of_peak": round(b64 / (mmean * 1e-3) / 1e9 / HBM_PEAK_GBPS, 3),
        }
        del m64, v64
        torch.cuda.empty_cache()
        # head_dim 256 (Gemma-style 16/8 heads), B=16, S=8192, on the same kernel
        c256 = type("Cfg", (), dict(B=16, Hq=16, Hkv=8, S=8192, D=256, n_sink=4, recent=64, mid=8192 - 68))
        m256 = build_instances(c256, "int4", dev, 1007, N_INSTANCES)
        v256 = [TieredDecodePlan(*pl._keep[:4], kernel=1) for pl in m256]
        mmean, vmean = graph_us(m256) * 1e-3, graph_us(v256) * 1e-3
        b256 = decode_bytes(c256, "int4")
        extra["c1_shape_d256_16_8_decode_int4"] = {
            "us": round(mmean * 1e3, 2), "us_portable_kernel": round(vmean * 1e3, 2), "bytes": b256,
            "GBps": round(b256 / (mmean * 1e-3) / 1e9, 1),
            "frac_of_peak": round(b256 / (mmean * 1e-3) / 1e9 / HBM_PEAK_GBPS, 3),
        }
        del m256, v256
        torch.cuda.empty_cache()
        # GQA 8 (Llama-3-70B / Qwen2-72B heads: 64 / 8) at config 1's batch and length
        g2, gg, gb = gqa7_decode_case(dev, B=16, S=8192, Hq=64, Hkv=8)
        g2mean = graph_us(g2) * 1e-3
        extra["b16_s8192_decode_gqa8_64_8_int4"] = {
            "us_int4_kernel": round(g2mean * 1e3, 2), "bytes": gb, "GBps": round(gb / (g2mean * 1e-3) / 1e9, 1),
            "frac_of_peak": round(gb / (g2mean * 1e-3) / 1e9 / HBM_PEAK_GBPS, 3),
        }
        del g2, gg
        torch.cuda.empty_cache()
        extra["copy_peak_GBps"] = round(copy_peak(dev, stream), 1)
        torch.cuda.empty_cache()
        c2 = CONFIGS[2]
        c2_traffic = {}
        if os.path.exists(TRAFFIC_FILE_C2):
            with open(TRAFFIC_FILE_C2) as f:
                c2_traffic = json.load(f)
        for fmt in ("asym42", "k4v2", "int4", "rot2"):  # asym42: the format BASELINE states for config 2
            pl = build_instances(c2, fmt, dev, 1002, N_INSTANCES)
            mean2 = graph_us(pl) * 1e-3
            b2 = decode_bytes(c2, fmt)
            extra[f"c2_32k_{fmt}"] = {
                "us": round(mean2 * 1e3, 2), "GBps": round(b2 / (mean2 * 1e-3) / 1e9, 1), "bytes": b2,
                "frac_of_peak": round(b2 / (mean2 * 1e-3) / 1e9 / HBM_PEAK_GBPS, 3),
            }
            tr = c2_traffic.get(f"c2_{fmt}")
            if tr is not None:  # rocprofv3 FETCH_SIZE + WRITE_SIZE of this format (profiles/decode_c2_32k.md)
                extra[f"c2_32k_{fmt}"]["traffic_ratio"] = tr["traffic_ratio"]
            if fmt == "rot2":  # the product path: unrotated q / sink / recent, R applied in the kernel
                extra[f"c2_32k_{fmt}"]["rotation"] = "in kernel (q R^T for the middle, middle output part times R)"
            del pl
            torch.cuda.empty_cache()

    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_call")

    line = {
        "metric": METRIC,
        "value": round(mean_ms * 1e3, 2),
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 K/V codes with fp16 scales and fp16 sink/recent tiers; QK^T of the codes on int8 "
        "MFMAs against the query times the K scales as a 16-bit fixed-point number in two 8-bit digits "
        "(exact int32 sums), PV on f16 MFMAs, fp32 softmax and accumulation, fp16 output",
        "data": "synthetic (seeded N(0,1) K*LogNormal(0,0.5) channel scales, V, Q)",
        "config": {
            "workload": "config 1: fused tiered decode, B=16, Hq=32, Hkv=8, D=128, S=8192 "
            "(4 fp16 sink + 8124 INT4 + 64 fp16 recent), reference INT4 format",
            "instances_rotated": N_INSTANCES,
            "settle_calls_before_timing": settled,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "algorithmic_bytes_per_call": nbytes,
            "timed": f"the K={args.steps} steps: HIP events around each of {replays} replay(s) of a HIP graph "
            f"of {calls} back-to-back calls (rotating over the {N_INSTANCES} instances) on the launch stream, "
            f"value = their total / K (one kernel: decode_packed_kernel<4,4,0,4,false,false,false>, split merge "
            f"fused); median_us: a separate statistics pass, the median over {STATS_REPLAYS} replays of a "
            f"{STATS_CALLS}-call graph (per call = replay / {STATS_CALLS}); eager_us_per_call: HIP events "
            "around each separately launched call",
            "replays": replays,
            "calls_per_replay": calls,
            "median_us": round(med_ms * 1e3, 2),
            "median_replays": STATS_REPLAYS,
            "eager_us_per_call": round(eager_mean_ms * 1e3, 2),
            "measured_read_ceiling_GBps": peak["GBps"],
            "frac_of_measured_read_ceiling": round(achieved / peak["GBps"], 3),
        },
        "extra": extra,
    }
    if cpu is not None:
        line["cpu_baseline"] = cpu
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
