"""Benchmark of the INT8 attention / Q4_K hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-secondary]

A "step" is one `_C.attn_int8_fwd` call (the prefill kernel alone: V is read
in place, no staging pass) at BASELINE config 2: B=1, Hq=32, Hkv=8, S=4096, D=128,
causal, on seeded synthetic N(0,1) fp16 Q/K/V quantised by the prologue
beforehand (inputs resident in HBM when the timed region starts).
`value` = algorithmic ops per step / step time, in TOPS, where the ops are
the reference harness's attention_flops(causal) = 2*B*H*S*S*D
(bench/harness.py:220-223 of the reference).

Also reported (under "secondary"): split-KV decode at config 3 and the Q4_K
GEMV at config 4 (M=1 and M=8), as HBM GB/s over their algorithmic bytes,
the public `attn_int8_fwd(q, k, v, causal=True)` at config 2 (prologue, gate
and kernel: what the reference's own benchmarks time),
the full-W8A8 prefill at config 5 (TOPS), and (under "cpu_baseline") the
numpy restatement of config 1 timed on the host cores. One JSON line is
printed on stdout.

Before the warmup steps the GPU runs ~0.3 s of untimed prefill calls: the
MI355X clocks ramp up over the first milliseconds of load, and the figures
are steady-state ones.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

PEAK_INT8_TOPS = 5000.0  # MI355X dense INT8 MFMA (vendor)
PEAK_HBM_GBS = 8000.0    # MI355X HBM3E

CFG2 = dict(B=1, Hq=32, Hkv=8, S=4096, D=128)
CFG2_OPS = 4 * 1 * 32 * 4096 * 4096 * 128 // 2  # 137,438,953,472


def _events_time(fn, iters, stream):
    """Average ms per call of fn(), HIP events on `stream` around the whole batch."""
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(iters):
        fn()
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / iters


def spin_up(fn, seconds=0.3):
    """Untimed calls until `seconds` of GPU work have run (clock ramp-up)."""
    torch.cuda.synchronize()
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


def bench_prefill(steps, warmup):
    from superl8_amd import _C, quant

    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(2)
    q = torch.randn(1, 32, 4096, 128, device=dev, dtype=torch.float16, generator=g)
    k = torch.randn(1, 8, 4096, 128, device=dev, dtype=torch.float16, generator=g)
    v = torch.randn(1, 8, 4096, 128, device=dev, dtype=torch.float16, generator=g)
    q_i8, qs, k_i8, ks, _ = quant.quantize_qk(q, k)
    qs, ks = qs.squeeze(-1).contiguous(), ks.squeeze(-1).contiguous()

    def step():
        return _C.attn_int8_fwd(q_i8, qs, k_i8, ks, v, True)

    spin_up(step)
    for _ in range(warmup):
        step()
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms = _events_time(step, steps, stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return ms, wall


def bench_public_prefill(iters=20):
    """The public API at config 2 from fp16 Q/K/V: fused K-smoothing + int8
    prologue, the on-device outlier gate (its flag read back by the host, as the
    reference's gate syncs), then the prefill kernel."""
    import superl8_amd as sl8

    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(2)
    q = torch.randn(1, 32, 4096, 128, device=dev, dtype=torch.float16, generator=g)
    k = torch.randn(1, 8, 4096, 128, device=dev, dtype=torch.float16, generator=g)
    v = torch.randn(1, 8, 4096, 128, device=dev, dtype=torch.float16, generator=g)
    fn = lambda: sl8.attn_int8_fwd(q, k, v, causal=True)  # noqa: E731
    spin_up(fn, 0.2)
    return _events_time(fn, iters, torch.cuda.current_stream())


def bench_decode(iters=20, ks16=False):
    """Config 3. ks16: the K cache's per-token scales stored as fp16 (the BASELINE
    config text; the reference contract is fp32)."""
    from superl8_amd import _C

    dev = "cuda"
    B, Hq, Hkv, N, D = 16, 32, 8, 32768, 128
    g = torch.Generator(device=dev).manual_seed(3)
    q = torch.randn(B * Hq, D, device=dev, dtype=torch.float16, generator=g)
    k = torch.randn(B * Hkv * N, D, device=dev, dtype=torch.float16, generator=g)
    q_i8, qs = _C.quantize_i8_rowwise(q)
    k_i8, ks = _C.quantize_i8_rowwise(k)  # per-token int8 K cache
    del k
    q_i8 = q_i8.reshape(B, Hq, 1, D)
    qs = (qs * (1.0 / np.sqrt(D) * np.log2(np.e))).reshape(B, Hq, 1).contiguous()
    k_i8 = k_i8.reshape(B, Hkv, N, D)
    ks = ks.reshape(B, Hkv, N)
    if ks16:
        ks = ks.half()
    v = torch.randn(B, Hkv, N, D, device=dev, dtype=torch.float16, generator=g)
    fn = lambda: _C.attn_int8_decode(q_i8, qs, k_i8, ks, v, 16)  # noqa: E731
    spin_up(fn, 0.2)
    ms = _events_time(fn, iters, torch.cuda.current_stream())
    nbytes = k_i8.numel() + ks.numel() * ks.element_size() + v.numel() * 2 + q_i8.numel() \
        + qs.numel() * 4 + B * Hq * D * 2
    return ms, nbytes


def bench_decode_kv8(iters=20, ns=16):
    """Decode over an int8 V cache (per-channel scale) at config 3's shape: K and V
    int8 [16, 8, 32768, 128], the row of reference attn_int8_decode_kv8 (survey next)."""
    from superl8_amd import _C

    dev = "cuda"
    B, Hq, Hkv, N, D = 16, 32, 8, 32768, 128
    g = torch.Generator(device=dev).manual_seed(7)
    q = torch.randn(B * Hq, D, device=dev, dtype=torch.float16, generator=g)
    k = torch.randn(B * Hkv * N, D, device=dev, dtype=torch.float16, generator=g)
    q_i8, qs = _C.quantize_i8_rowwise(q)
    k_i8, ks = _C.quantize_i8_rowwise(k)
    del k
    q_i8 = q_i8.reshape(B, Hq, 1, D)
    qs = (qs * (1.0 / np.sqrt(D) * np.log2(np.e))).reshape(B, Hq, 1).contiguous()
    k_i8 = k_i8.reshape(B, Hkv, N, D)
    ks = ks.reshape(B, Hkv, N)
    v = torch.randn(B, Hkv, N, D, device=dev, dtype=torch.float16, generator=g)
    v_i8, vs = _C.quantize_v_perchannel(v)
    del v
    vs = vs.reshape(B, Hkv, D).contiguous()
    fn = lambda: _C.attn_int8_decode_kv8(q_i8, qs, k_i8, ks, v_i8, vs, ns)  # noqa: E731
    spin_up(fn, 0.2)
    ms = _events_time(fn, iters, torch.cuda.current_stream())
    nbytes = k_i8.numel() + ks.numel() * 4 + v_i8.numel() + vs.numel() * 4 + q_i8.numel() \
        + qs.numel() * 4 + B * Hq * D * 2
    return ms, nbytes


def bench_paged_decode(iters=20, bs=16):
    """Paged int8 KV decode at config 3's shape: 16 sequences of 32768 keys in
    16-key blocks scattered over the pool by a shuffled block table, per-token
    K and V scales (reference attn_paged_decode)."""
    from superl8_amd import _C

    dev = "cuda"
    B, Hq, Hkv, N, D = 16, 32, 8, 32768, 128
    g = torch.Generator(device=dev).manual_seed(8)
    nblk = B * N // bs
    kc = torch.randint(-127, 128, (nblk, Hkv, bs, D), device=dev, dtype=torch.int8, generator=g)
    vc = torch.randint(-127, 128, (nblk, Hkv, bs, D), device=dev, dtype=torch.int8, generator=g)
    ks = torch.rand(nblk, Hkv, bs, device=dev, generator=g) * 0.02 + 1e-3
    vs = torch.rand(nblk, Hkv, bs, device=dev, generator=g) * 0.02 + 1e-3
    bt = torch.randperm(nblk, device=dev, generator=g).to(torch.int32).reshape(B, N // bs)
    ctx = torch.full((B,), N, device=dev, dtype=torch.int32)
    q = torch.randint(-127, 128, (B, Hq, 1, D), device=dev, dtype=torch.int8, generator=g)
    qs = torch.rand(B, Hq, 1, device=dev, generator=g) * 0.01 + 1e-3
    fn = lambda: _C.attn_paged_decode(q, qs, kc, ks, vc, vs, bt, ctx, bs, N, 16)  # noqa: E731
    spin_up(fn, 0.2)
    ms = _events_time(fn, iters, torch.cuda.current_stream())
    nbytes = kc.numel() + vc.numel() + (ks.numel() + vs.numel()) * 4 + bt.numel() * 4 \
        + q.numel() + qs.numel() * 4 + B * Hq * D * 2
    return ms, nbytes


def bench_paged_decode_k8v3(iters=20, bs=16, D=128):
    """K8V3 paged decode at config 3's shape (D = 256: the same layout with the
    head dim of the reference's K8V3 models): int8 K with per-token scales and
    3-bit Lloyd-Max V (packed codes + per-128-channel norms + codebook), 16-key
    blocks scattered by a shuffled block table (reference attn_paged_decode_k8v3)."""
    from superl8_amd import _C
    from superl8_amd.quant.lloydmax import gaussian_codebook

    dev = "cuda"
    B, Hq, Hkv, N = 16, 32, 8, 32768
    g = torch.Generator(device=dev).manual_seed(10)
    nblk = B * N // bs
    kc = torch.randint(-127, 128, (nblk, Hkv, bs, D), device=dev, dtype=torch.int8, generator=g)
    ks = torch.rand(nblk, Hkv, bs, device=dev, generator=g) * 0.02 + 1e-3
    vp = torch.randint(-2 ** 31, 2 ** 31 - 1, (nblk, Hkv, bs, 3 * D // 32), device=dev,
                       dtype=torch.int32, generator=g)
    vn = torch.rand(nblk, Hkv, bs, D // 128, device=dev, generator=g) * 20 + 1
    cb = gaussian_codebook(3, 128).to(dev)
    bt = torch.randperm(nblk, device=dev, generator=g).to(torch.int32).reshape(B, N // bs)
    ctx = torch.full((B,), N, device=dev, dtype=torch.int32)
    q = torch.randint(-127, 128, (B, Hq, 1, D), device=dev, dtype=torch.int8, generator=g)
    qs = torch.rand(B, Hq, 1, device=dev, generator=g) * 0.01 + 1e-3
    fn = lambda: _C.attn_paged_decode_k8v3(q, qs, kc, ks, vp, vn, cb, bt, ctx, bs, N, 16)  # noqa: E731
    spin_up(fn, 0.2)
    ms = _events_time(fn, iters, torch.cuda.current_stream())
    nbytes = kc.numel() + ks.numel() * 4 + vp.numel() * 4 + vn.numel() * 4 + bt.numel() * 4 \
        + q.numel() + qs.numel() * 4 + B * Hq * D * 2
    return ms, nbytes


def bench_gemm_prefill(M=512, iters=10, fmt="q4k"):
    """k-quant prefill GEMM (M > 16: the tiled MFMA kernel) on config 4's shape."""
    from superl8_amd import _C

    dev = "cuda"
    N, K = 17408, 5120
    w = _kquant_weights(fmt, N, K, 4).to(dev)
    g = torch.Generator(device=dev).manual_seed(9)
    x = torch.randn(M, K, device=dev, dtype=torch.float16, generator=g)
    x_i8, xs = _C.quantize_i8_rowwise(x)
    op = getattr(_C, f"gemm_{fmt}")
    fn = lambda: op(x_i8, xs, w)  # noqa: E731
    spin_up(fn, 0.1)
    ms = _events_time(fn, iters, torch.cuda.current_stream())
    return ms, 2 * M * N * K


def bench_prologue(iters=20):
    """Attention prologue at config 2: the fused two-launch sl8_quantize_qk with the
    outlier gate, and the separate kernels it replaces (K mean, Q and K quantise,
    gate). Algorithmic bytes: Q and K read once, codes and scales written once."""
    from superl8_amd import _C
    from superl8_amd.quant import LOG2E

    dev = "cuda"
    B, Hq, Hkv, S, D = 1, 32, 8, 4096, 128
    g = torch.Generator(device=dev).manual_seed(3)
    q = torch.randn(B, Hq, S, D, device=dev, dtype=torch.float16, generator=g)
    k = torch.randn(B, Hkv, S, D, device=dev, dtype=torch.float16, generator=g)
    mul = LOG2E / D ** 0.5
    fused = lambda: _C.quantize_qk_fused(q, k, mul, 12.0)  # noqa: E731

    def separate():
        m = _C.k_mean(k)
        _C.quantize_rows_centered(q, None, mul)
        _C.quantize_rows_centered(k, m, 1.0)
        _C.q_outlier_gate(q, 12.0)

    st = torch.cuda.current_stream()
    spin_up(fused, 0.1)
    fms = _events_time(fused, iters, st)
    sms = _events_time(separate, iters, st)
    nbytes = (q.numel() + k.numel()) * 3 + (B * Hq * S + B * Hkv * S) * 4
    return fms, sms, nbytes


def bench_w8a8(iters=5, per_wave=False, exact_pv=False):
    """Full-W8A8 prefill at BASELINE config 5: Q/K/V [2, 16|2, 8192, 256], causal,
    1% of Q/K channels (3 of 256, fixed) scaled by 20, V per-channel int8.
    per_wave: Q/K quantised per wavefront tile (32 queries / 64 keys), the config
    text, instead of the reference's per row (the kernel is the same).
    exact_pv: the reference's per-warp arithmetic exactly (int32 P.V per half)."""
    from superl8_amd import _C, quant

    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(6)
    B, Hq, Hkv, S, D = 2, 16, 2, 8192, 256
    q = torch.randn(B, Hq, S, D, device=dev, dtype=torch.float16, generator=g)
    k = torch.randn(B, Hkv, S, D, device=dev, dtype=torch.float16, generator=g)
    v = torch.randn(B, Hkv, S, D, device=dev, dtype=torch.float16, generator=g)
    ch = torch.tensor([17, 101, 203], device=dev)
    q[..., ch] *= 20
    k[..., ch] *= 20
    qfn = quant.quantize_qk_per_wave if per_wave else quant.quantize_qk
    q_i8, qs, k_i8, ks, _ = qfn(q, k)
    qs, ks = qs.squeeze(-1).contiguous(), ks.squeeze(-1).contiguous()
    v_i8, vs = _C.quantize_v_perchannel(v)
    vs = vs.reshape(B, Hkv, D).contiguous()
    del q, k, v
    fn = lambda: _C.attn_w8a8_fwd(q_i8, qs, k_i8, ks, v_i8, vs, True, exact_pv=exact_pv)  # noqa: E731
    spin_up(fn, 0.2)
    ms = _events_time(fn, iters, torch.cuda.current_stream())
    ops = 4 * B * Hq * S * S * D // 2
    return ms, ops


def _kquant_weights(fmt, N, K, seed):
    """Synthetic native GGUF bytes (data generators only; nothing here is measured)."""
    from oracle import kquant as okq
    from oracle import q4k as oq

    gen = {"q4k": oq.random_weights, "q5k": okq.q5k_random, "q6k": okq.q6k_random}[fmt]
    return torch.from_numpy(gen(N, K, seed=seed))


KQ_BYTES = {"q4k": 144, "q5k": 176, "q6k": 210}


def bench_gemv(M, iters_graph=10, copies=8, fmt="q4k", xblock=False):
    """xblock: activations int8 per 256-element block with one fp32 scale each
    (x_scale [M, K/256], the BASELINE config 4 text) instead of per row."""
    from superl8_amd import _C

    dev = "cuda"
    N, K = 17408, 5120
    op = getattr(_C, f"gemm_decode_{fmt}")
    base = _kquant_weights(fmt, N, K, 4).to(dev)
    ws = [base] + [base.roll(i * 1, 0).contiguous() for i in range(1, copies)]  # > 256 MB MALL
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(M, K, device=dev, dtype=torch.float16, generator=g)
    x_i8, xs = _C.quantize_i8_blockwise(x, 256) if xblock else _C.quantize_i8_rowwise(x)
    for w in ws:
        op(x_i8, xs, w)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    per_graph = 8 * copies
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            for i in range(per_graph):
                op(x_i8, xs, ws[i % copies])
    for _ in range(2):
        graph.replay()
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    ms = _events_time(graph.replay, iters_graph, cur) / per_graph
    nbytes = N * (K // 256) * KQ_BYTES[fmt] + M * K + xs.numel() * 4 + M * N * 2
    return ms, nbytes


def bench_copy(nbytes=256 << 20, iters=20):
    """A plain device-to-device copy (torch): the practical HBM ceiling on this box.
    Returns GB/s counting bytes read + bytes written."""
    src = torch.empty(nbytes, device="cuda", dtype=torch.uint8)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    ms = _events_time(lambda: dst.copy_(src), iters, torch.cuda.current_stream())
    return 2 * nbytes / (ms * 1e-3) / 1e9


def cpu_baseline(budget_s=12.0):
    """numpy restatement (oracle) of config 1: prologue + causal attention,
    B=1, H=8, S=512, D=64, timed on this host; trimmed median over repeats."""
    from oracle import attention as oa
    from oracle import quant as oqn

    # All host cores, as the reference's harness asks (torch.set_num_threads(
    # os.cpu_count())); the numpy oracle's BLAS pool gets the same limit. The GPU
    # box caps OMP_NUM_THREADS, so the pool that actually ran is reported too.
    ncpu = os.cpu_count() or 1
    torch.set_num_threads(ncpu)
    from threadpoolctl import threadpool_info, threadpool_limits
    limiter = threadpool_limits(limits=ncpu)
    threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    rng = np.random.default_rng(1)
    q, k, v = (rng.standard_normal((1, 8, 512, 64)).astype(np.float16) for _ in range(3))

    def run():
        q_i8, qs, k_i8, ks, _ = oqn.quantize_qk(q, k)
        return oa.attn_int8_fwd(q_i8, qs, k_i8, ks, v.astype(np.float32), True)

    run()
    samples = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end and len(samples) < 200:
        t0 = time.perf_counter()
        run()
        samples.append(time.perf_counter() - t0)
    samples.sort()
    k_trim = max(1, len(samples) // 10) if len(samples) > 4 else 0
    trimmed = samples[k_trim:len(samples) - k_trim] if k_trim else samples
    med = float(np.median(trimmed))
    ops = 4 * 1 * 8 * 512 * 512 * 64 // 2
    secondary = cpu_secondary()
    limiter.unregister()
    return {
        "value": round(ops / med / 1e9, 3),
        "unit": "GOPS",
        "cores": int(threads),
        "os_cpu_count": int(ncpu),
        "torch_threads": int(torch.get_num_threads()),
        "kind": "port",
        "sample": f"config 1 (B1 H8 S512 D64 causal, quantize_qk + attention), numpy oracle, "
                  f"{len(samples)} runs, trimmed median {med * 1e3:.1f} ms/run",
        "secondary": secondary,
    }


def _median_time(fn, runs):
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def cpu_secondary(runs=3):
    """The decode and GEMV lines' CPU counterparts (numpy oracle, same byte
    accounting as the GPU lines): config 3 decode on one of its 16 sequences
    (the per-sequence work is identical), config 4's Q4_K GEMV at full size."""
    from oracle import attention as oa
    from oracle import q4k as oq
    from oracle import quant as oqn

    out = {}
    rng = np.random.default_rng(3)
    Hq, Hkv, N, D = 32, 8, 32768, 128
    q = rng.integers(-127, 128, (1, Hq, D)).astype(np.int8)
    qs = np.full((1, Hq), 1e-3, np.float32)
    k = rng.integers(-127, 128, (1, Hkv, N, D)).astype(np.int8)
    ks = (rng.random((1, Hkv, N)) * 0.02).astype(np.float32)
    v16 = rng.standard_normal((1, Hkv, N, D)).astype(np.float16)
    v = v16.astype(np.float32)  # fp16 values; the conversion is outside the timing
    t = _median_time(lambda: oa.attn_int8_decode(q, qs, k, ks, v, 16), runs)
    nbytes = k.size + ks.size * 4 + v16.size * 2 + q.size + qs.size * 4 + Hq * D * 2
    out["attn_int8_decode_cfg3_one_sequence"] = {
        "ms": round(t * 1e3, 1), "GB/s": round(nbytes / t / 1e9, 3), "bytes": int(nbytes)}
    del k, v, v16
    N4, K4 = 17408, 5120
    w = oq.random_weights(N4, K4, seed=4)
    for M in (1, 8):
        x = rng.standard_normal((M, K4)).astype(np.float16).astype(np.float32)
        xi, xsc = oqn.quantize_rows(x)
        t = _median_time(lambda: oq.gemv(xi, xsc, w, K4), runs)
        nbytes = N4 * (K4 // 256) * 144 + M * K4 + M * 4 + M * N4 * 2
        out[f"gemm_decode_q4k_cfg4_m{M}"] = {
            "ms": round(t * 1e3, 1), "GB/s": round(nbytes / t / 1e9, 3), "bytes": int(nbytes)}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="summarise a rocprofv3 --kernel-trace CSV of a `--no-secondary` run "
                         "(the timed calls = the prefill kernel's last --steps dispatches) "
                         "and exit; runs without a GPU")
    ap.add_argument("--pmc-summary", metavar="COUNTER_COLLECTION_CSV",
                    help="summarise a rocprofv3 --pmc CSV: per kernel, the median (and max) over "
                         "its dispatches of each counter summed over the dispatch's rows; exits")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 256 MiB device copy (scale for PMC byte counters)")
    args = ap.parse_args()
    if args.trace_summary:
        print(trace_summary(args.trace_summary, args.steps))
        return
    if args.pmc_summary:
        print(pmc_summary(args.pmc_summary))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(prefill and decode would shard over batch x KV-head groups with no exchange "
              "beyond the decode's LSE merge); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        src = torch.empty(256 << 20, device="cuda", dtype=torch.uint8)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    ms, wall = bench_prefill(args.steps, args.warmup)
    tops = CFG2_OPS / (ms * 1e-3) / 1e12
    out = {
        "metric": "INT8 attn fwd TOPS (%MFMA peak); decode + Q4_K GEMV HBM GB/s (%peak)",
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 QK^T / fp16 PV",
        "data": "synthetic (seeded N(0,1) fp16 Q/K/V, int8 per-row quantised with K smoothing)",
        "config": {"workload": "attn_int8_fwd prefill, BASELINE config 2", "batch": 1,
                   "heads_q": 32, "heads_kv": 8, "seq_len": 4096, "head_dim": 128,
                   "causal": True},
        "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": PEAK_INT8_TOPS,
                     "unit": "TOP/s", "frac": round(tops / PEAK_INT8_TOPS, 4),
                     "traffic": _traffic("attn_int8_fwd")},
    }
    if not args.no_secondary:
        sec = {}
        pub = bench_public_prefill()
        sec["attn_int8_fwd_public_api_cfg2"] = {
            "us": round(pub * 1e3, 2), "TOPS": round(CFG2_OPS / (pub * 1e-3) / 1e12, 1),
            "frac_int8_peak": round(CFG2_OPS / (pub * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4),
            "includes": "fused prologue + outlier gate + host flag read + kernel"}
        dms, dbytes = bench_decode()
        gbs = dbytes / (dms * 1e-3) / 1e9
        sec["attn_int8_decode_cfg3"] = {"us": round(dms * 1e3, 2), "GB/s": round(gbs, 1),
                                        "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                                        "bytes": dbytes}
        dms, dbytes = bench_decode(ks16=True)
        gbs = dbytes / (dms * 1e-3) / 1e9
        sec["attn_int8_decode_cfg3_fp16_kscale"] = {"us": round(dms * 1e3, 2), "GB/s": round(gbs, 1),
                                                    "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                                                    "bytes": dbytes}
        kms, kbytes = bench_decode_kv8()
        gbs = kbytes / (kms * 1e-3) / 1e9
        sec["attn_int8_decode_kv8_cfg3shape"] = {"us": round(kms * 1e3, 2), "GB/s": round(gbs, 1),
                                                 "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                                                 "bytes": kbytes}
        pms, pbytes = bench_paged_decode()
        gbs = pbytes / (pms * 1e-3) / 1e9
        sec["attn_paged_decode_cfg3shape_bs16"] = {"us": round(pms * 1e3, 2), "GB/s": round(gbs, 1),
                                                   "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                                                   "bytes": pbytes}
        for dk, key in ((128, "attn_paged_decode_k8v3_cfg3shape_bs16"),
                        (256, "attn_paged_decode_k8v3_cfg3layout_d256_bs16")):
            pms, pbytes = bench_paged_decode_k8v3(D=dk)
            gbs = pbytes / (pms * 1e-3) / 1e9
            sec[key] = {"us": round(pms * 1e3, 2), "GB/s": round(gbs, 1),
                        "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": pbytes}
        for M in (1, 8):
            gms, gbytes = bench_gemv(M)
            gbs = gbytes / (gms * 1e-3) / 1e9
            sec[f"gemm_decode_q4k_cfg4_m{M}"] = {"us": round(gms * 1e3, 2), "GB/s": round(gbs, 1),
                                                 "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                                                 "bytes": gbytes}
        for M in (1, 8):
            gms, gbytes = bench_gemv(M, xblock=True)
            gbs = gbytes / (gms * 1e-3) / 1e9
            sec[f"gemm_decode_q4k_cfg4_m{M}_xblock256"] = {
                "us": round(gms * 1e3, 2), "GB/s": round(gbs, 1),
                "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": gbytes}
        pms2, pops = bench_gemm_prefill()
        pt = pops / (pms2 * 1e-3) / 1e12
        sec["gemm_q4k_prefill_m512_cfg4w"] = {"us": round(pms2 * 1e3, 1), "TOPS": round(pt, 1),
                                              "frac_int8_peak": round(pt / PEAK_INT8_TOPS, 4),
                                              "ops": pops}
        for fmt in ("q5k", "q6k"):
            for M in (1, 8):
                gms, gbytes = bench_gemv(M, fmt=fmt)
                gbs = gbytes / (gms * 1e-3) / 1e9
                sec[f"gemm_decode_{fmt}_cfg4shape_m{M}"] = {
                    "us": round(gms * 1e3, 2), "GB/s": round(gbs, 1),
                    "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": gbytes}
            pms2, pops = bench_gemm_prefill(fmt=fmt)
            pt = pops / (pms2 * 1e-3) / 1e12
            sec[f"gemm_{fmt}_prefill_m512_cfg4shape"] = {
                "us": round(pms2 * 1e3, 1), "TOPS": round(pt, 1),
                "frac_int8_peak": round(pt / PEAK_INT8_TOPS, 4), "ops": pops}
        fms, sms, pb = bench_prologue()
        gbs = pb / (fms * 1e-3) / 1e9
        sec["prologue_quantize_qk_gate_cfg2"] = {"us": round(fms * 1e3, 2), "GB/s": round(gbs, 1),
                                                 "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                                                 "bytes": pb,
                                                 "separate_kernels_us": round(sms * 1e3, 2)}
        wms, wops = bench_w8a8()
        wt = wops / (wms * 1e-3) / 1e12
        sec["attn_w8a8_fwd_cfg5"] = {"us": round(wms * 1e3, 1), "TOPS": round(wt, 1),
                                     "frac_int8_peak": round(wt / PEAK_INT8_TOPS, 4), "ops": wops}
        wms, wops = bench_w8a8(per_wave=True)
        wt = wops / (wms * 1e-3) / 1e12
        sec["attn_w8a8_fwd_cfg5_per_wave_qk"] = {"us": round(wms * 1e3, 1), "TOPS": round(wt, 1),
                                                 "frac_int8_peak": round(wt / PEAK_INT8_TOPS, 4),
                                                 "ops": wops}
        wms, wops = bench_w8a8(exact_pv=True)
        wt = wops / (wms * 1e-3) / 1e12
        sec["attn_w8a8_fwd_cfg5_exact_pv"] = {"us": round(wms * 1e3, 1), "TOPS": round(wt, 1),
                                              "frac_int8_peak": round(wt / PEAK_INT8_TOPS, 4),
                                              "ops": wops,
                                              "mode": "per-warp P, exact int32 P.V per 32-key half"}
        sec["hbm_copy_256MiB_GBps"] = round(bench_copy(), 1)
        out["secondary"] = sec
    if not args.no_cpu:
        cb = cpu_baseline()
        # GPU-over-CPU ratios of the same metric (a baseline, not a target)
        cb["gpu_over_cpu"] = {"attn_int8_fwd": round(out["value"] * 1e3 / cb["value"], 1)}
        sec = out.get("secondary", {})
        for key, gkey in (("attn_int8_decode_cfg3_one_sequence", "attn_int8_decode_cfg3"),
                          ("gemm_decode_q4k_cfg4_m1", "gemm_decode_q4k_cfg4_m1"),
                          ("gemm_decode_q4k_cfg4_m8", "gemm_decode_q4k_cfg4_m8")):
            if gkey in sec:
                cb["gpu_over_cpu"][gkey] = round(sec[gkey]["GB/s"] / cb["secondary"][key]["GB/s"], 1)
        out["cpu_baseline"] = cb
    print(json.dumps(out), flush=True)


PREFILL_KERNEL = "attn_fwd_wide_kernel<128, true, 0, false, 1, 8, false, false>"


def _short_kernel_name(name: str) -> str:
    """'void sl8::(anonymous namespace)::k<..>(sl8::..)' -> 'k<..>' (full template
    arguments kept)."""
    import re

    name = re.sub(r"^void ", "", name)
    name = re.sub(r"sl8::\(anonymous namespace\)::", "", name)
    name = name.replace("(anonymous namespace)", "anon")
    depth, end = 0, len(name)
    for i, ch in enumerate(name):  # cut the parameter list after the template arguments
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            end = i
            break
    return name[:end]


def trace_summary(path: str, steps: int) -> str:
    """Markdown table from a rocprofv3 kernel-trace CSV. Every dispatch is listed
    per kernel (count, mean, median, min, max); for the config 2 prefill kernel the
    timed calls of `bench.py --no-secondary --steps K` are its last K dispatches
    (the spin-up and warmup calls come first), reported separately."""
    import csv

    by = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            n = _short_kernel_name(r["Kernel_Name"])
            t0, t1 = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
            by.setdefault(n, []).append((t0, (t1 - t0) / 1e3))
    lines = ["| kernel | calls | mean us | median us | min us | max us |", "|---|---|---|---|---|---|"]
    for n, v in sorted(by.items(), key=lambda kv: -sum(d for _, d in kv[1])):
        d = [x for _, x in v]
        nm = n if len(n) <= 120 else n[:117] + "..."
        lines.append(f"| {nm} | {len(d)} | {np.mean(d):.2f} | {np.median(d):.2f} | {min(d):.2f} | "
                     f"{max(d):.2f} |")
    if PREFILL_KERNEL in by:
        v = sorted(by[PREFILL_KERNEL])[-steps:]
        d = [x for _, x in v]
        span = (v[-1][0] - v[0][0]) / 1e3 / max(1, len(v) - 1) if len(v) > 1 else float("nan")
        lines += ["", f"Timed calls ({len(d)}: the last {steps} dispatches of `{PREFILL_KERNEL}`): "
                      f"mean {np.mean(d):.2f} us, median {np.median(d):.2f} us, min {min(d):.2f}, "
                      f"max {max(d):.2f}; start-to-start spacing {span:.2f} us."]
    return "\n".join(lines)


def pmc_summary(path: str) -> str:
    """Markdown table from a rocprofv3 --pmc counter-collection CSV: per kernel and
    counter, the value of each dispatch (its rows summed: one per XCD or
    instance) and the median and max over the dispatches."""
    import csv

    agg = {}
    for r in csv.DictReader(open(path)):
        n = _short_kernel_name(r["Kernel_Name"])
        d = agg.setdefault(n, {}).setdefault(r["Counter_Name"], {})
        d[r["Dispatch_Id"]] = d.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
    counters = sorted({c for v in agg.values() for c in v})
    lines = ["| kernel | dispatches | " + " | ".join(f"{c} median / max" for c in counters) + " |",
             "|---|---|" + "---|" * len(counters)]
    for n, cs in sorted(agg.items()):
        nd = max(len(v) for v in cs.values())
        cells = []
        for c in counters:
            v = list(cs.get(c, {}).values())
            cells.append(f"{np.median(v):.6g} / {max(v):.6g}" if v else "-")
        lines.append(f"| {n if len(n) <= 120 else n[:117] + '...'} | {nd} | " + " | ".join(cells) + " |")
    return "\n".join(lines)


def _traffic(kernel: str):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if present."""
    path = os.path.join(HERE, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(kernel)
    except (OSError, ValueError):
        return None


if __name__ == "__main__":
    main()
