#!/usr/bin/env python3
"""Decode-attention benchmark on one MI355X.

A step is one decode step of one attention layer: quantize-append one new K/V
token into the int8 cache and attend 32 query heads (GQA 8:1 over 4 KV heads,
head_dim 128) over every cached token, in one fused launch
(``rec_decode_append_attn``).  The headline workload is a 32K-token context;
the same run measures a 252K (258,048-token) context.

Inputs are resident in HBM before timing starts.  To keep the 256 MB
Infinity Cache (MALL) from serving the KV cache, consecutive steps rotate over
independent cache instances totalling more than 1 GB (32 x 34 MB at 32K,
4 x 268 MB at 252K).  Each instance starts ``n`` tokens short of the context
and grows by one token per step it serves.

Timing: W eager warm-up steps, then K steps captured in one HIP graph, one
untimed warm replay, then five replays of exactly K steps each between
synchronisations (HIP events on the launch stream); the headline is their
median.  A
step is two launches: the fused append + attention kernel and the split
merge.  For the roofline, K launches of the attention kernel alone
(``rec_decode_partial``) are captured and timed the same way.  Algorithmic
bytes per step are the K/V codes and scales of all T tokens read once, the
query read, the fp32 output written and the appended token read and written.

The CPU baseline times the oracle's split-K restatement (chunked
dequantization, float32 attention with sinks, merge) on the host over a
bounded sample of the same 32K workload.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "decode-attn HBM GB/s (% of peak) and µs/step per layer at 32K and 252K ctx"
HQ, HKV, D = 32, 4, 128
SCALE = 1.0 / np.sqrt(D)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_kernel_traffic.json")
CALIB_BYTES = 256 << 20


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


AFFINE = "affine"  # MLX-style affine group 64: 8-bit keys, 4-bit values, bf16 scale + bias


def row_bytes(bits, is_v=False):
    """Bytes per token per KV head: codes + scales (+ zero-points or biases)."""
    if bits == AFFINE:
        return (D // 2 if is_v else D) + 8  # codes + 2 groups x (bf16 scale + bf16 bias)
    return D + 2 if bits == 8 else D // 2 + 16  # codes + fp16 scale (+ zero-points)


def step_bytes(T, B=1, k_bits=8, v_bits=8, output=True, hq=HQ, hkv=HKV):
    """Algorithmic HBM bytes of one decode step over T tokens: K/V codes and
    scales read once, query read, appended token read (fp16) and written
    (codes + scale), fp32 output written (by the merge when output=False)."""
    kv = B * T * hkv * (row_bytes(k_bits) + row_bytes(v_bits, True))
    q = B * hq * D * 2
    out = B * hq * D * 4 if output else 0
    append = B * hkv * (2 * D * 2 + row_bytes(k_bits) + row_bytes(v_bits, True))
    return kv + q + out + append


class DecodeWorkload:
    """R cache instances of one context length plus a pool of new tokens."""

    def __init__(self, T, R, total_steps, seed, splits=0, bits=8, kind="outliers", frac=0.01, batch=1,
                 hq=HQ, hkv=HKV):
        import torch

        import rec_amd
        from rec_amd import synthetic

        self.torch, self.lib = torch, rec_amd.library()
        self.T, self.R, self.splits, self.bits, self.B = T, R, splits, bits, batch
        self.hq, self.hkv = hq, hkv
        B, HQ, HKV = batch, hq, hkv
        counts = [len(range(i, total_steps, R)) for i in range(R)]
        self.caches = []
        for i in range(R):
            T0 = T - counts[i]
            c = (rec_amd.QuantizedKVCache(64, 8, 4, max_tokens=T) if bits == AFFINE
                 else rec_amd.QuantizedKVCache(32, bits, bits, max_tokens=T))
            # the affine cache of a bf16 model (the reference's): scales and biases in bf16
            kdt = torch.bfloat16 if bits == AFFINE else torch.float16
            k = synthetic.kv((B, HKV, T0, D), seed + 2 * i, kind=kind, frac=frac, dtype=kdt)
            v = synthetic.kv((B, HKV, T0, D), seed + 2 * i + 1, kind=kind, frac=frac, dtype=kdt)
            c.update_and_fetch(k, v)
            del k, v
            self.caches.append(c)
        P = 16
        self.pool = [
            (
                synthetic.query(B, HQ, 1, seed + 1000 + j)[:, :, 0].contiguous(),
                synthetic.kv((B, HKV, 1, D), seed + 2000 + j),
                synthetic.kv((B, HKV, 1, D), seed + 3000 + j),
            )
            for j in range(P)
        ]
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.sinks = torch.randn(HQ, generator=g, device="cuda")
        self.out = torch.empty((B, HQ, D), dtype=torch.float32, device="cuda")
        self.ws = torch.zeros(self.lib.rec_decode_workspace_bytes(B, HKV, 256), dtype=torch.uint8, device="cuda")
        self.step_T = []
        torch.cuda.synchronize()

    def step(self, s, partial_only=False):
        """Launch one decode step on the current stream: the fused
        append+attention kernel and the split merge, or (partial_only) the
        append+attention kernel alone, for timing that kernel by itself."""
        from rec_amd import _lib

        c = self.caches[s % self.R]
        q, kn, vn = self.pool[s % len(self.pool)]
        T = c.offset + 1
        kc, ks, kz = c.keys
        vc, vs, vz = c.values
        stream = self.torch.cuda.current_stream().cuda_stream
        fn = self.lib.rec_decode_partial if partial_only else self.lib.rec_decode_append_attn
        kcode, vcode = (kv.code for kv in c.keys_and_values())  # the formats the cache holds
        rc = fn(
            q.data_ptr(), _lib.REC_F16, q.stride(0), q.stride(1),
            kn.data_ptr(), vn.data_ptr(), _lib.REC_F16, kn.stride(0), kn.stride(1), vn.stride(0), vn.stride(1),
            kcode, kc.data_ptr(), ks.data_ptr(), None if kz is None else kz.data_ptr(),
            vcode, vc.data_ptr(), vs.data_ptr(), None if vz is None else vz.data_ptr(),
            self.sinks.data_ptr(), SCALE, self.B, self.hq, self.hkv, D, T, c.capacity, self.splits,
            self.ws.data_ptr(), self.ws.numel(), _lib.REC_F32, self.out.data_ptr(), stream,
        )
        _lib.check(rc, "decode step")
        c.offset = T
        return T

    def attend_only(self, s):
        """rec_decode_attn over the cached tokens, no append (the attention half
        of an unfused step); the offset does not move."""
        from rec_amd import _lib

        c = self.caches[s % self.R]
        q = self.pool[s % len(self.pool)][0]
        kc, ks, kz = c.keys
        vc, vs, vz = c.values
        kcode, vcode = (kv.code for kv in c.keys_and_values())  # the formats the cache holds
        rc = self.lib.rec_decode_attn(
            q.data_ptr(), _lib.REC_F16, q.stride(0), q.stride(1),
            kcode, kc.data_ptr(), ks.data_ptr(), None if kz is None else kz.data_ptr(),
            vcode, vc.data_ptr(), vs.data_ptr(), None if vz is None else vz.data_ptr(),
            self.sinks.data_ptr(), SCALE, None, 0, 0, 0, 0, self.B, self.hq, self.hkv, D, c.offset, c.capacity,
            self.splits,
            self.ws.data_ptr(), self.ws.numel(), _lib.REC_F32, self.out.data_ptr(),
            self.torch.cuda.current_stream().cuda_stream,
        )
        _lib.check(rc, "decode attention")

    def append_only(self, s):
        """rec_kv_append of one token at the last cached position (the append
        half of an unfused step); the offset does not move."""
        from rec_amd import _lib

        c = self.caches[s % self.R]
        _, kn, vn = self.pool[s % len(self.pool)]
        kc, ks, kz = c.keys
        vc, vs, vz = c.values
        kcode, vcode = (kv.code for kv in c.keys_and_values())  # the formats the cache holds
        rc = self.lib.rec_kv_append(
            kn.data_ptr(), vn.data_ptr(), _lib.REC_F16, kn.stride(0), kn.stride(1), kn.stride(2),
            vn.stride(0), vn.stride(1), vn.stride(2),
            kcode, kc.data_ptr(), ks.data_ptr(), None if kz is None else kz.data_ptr(),
            vcode, vc.data_ptr(), vs.data_ptr(), None if vz is None else vz.data_ptr(),
            self.B, self.hkv, 1, D, c.offset - 1, c.capacity, self.torch.cuda.current_stream().cuda_stream,
        )
        _lib.check(rc, "append")


def _queue_ahead(torch):
    """Keep the GPU busy for ~100 us before a timed region, so the host has
    enqueued the start event and the graph's launches by the time the GPU
    reaches them: the region then times the steps, not the host's submission
    latency.  Runs before the start event, outside the timed region."""
    if hasattr(torch.cuda, "_sleep"):
        torch.cuda._sleep(200_000)  # GPU clock cycles of a one-thread spin kernel


class _TimingEvents:
    """A pair of HIP timing events created with hipEventDisableSystemFence,
    recorded on torch's current stream.  By default recording an event
    releases and acquires at system scope (an L2 writeback and invalidate),
    which adds a fixed ~12 us to every timed replay and slows the work right
    after the start event; events used only for timing do not need it (the
    device is synchronised before the elapsed time is read).  Bound through
    the HIP runtime torch has loaded."""

    FLAGS = 0x20000000  # hipEventDisableSystemFence

    @staticmethod
    def _loaded_runtime():
        """The HIP runtime file this process has mapped (torch's), so that
        the events and the work share one runtime."""
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64" in line:
                    return line.split()[-1]
        raise RuntimeError("the HIP runtime is not loaded (initialise the GPU first)")

    def __init__(self):
        hip = ctypes.CDLL(self._loaded_runtime())
        hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.hip = hip
        self.ev = [ctypes.c_void_p(), ctypes.c_void_p()]
        for e in self.ev:
            self._check(hip.hipEventCreateWithFlags(ctypes.byref(e), self.FLAGS), "hipEventCreateWithFlags")

    @staticmethod
    def _check(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed with HIP error {rc}")

    def record(self, i, stream):
        self._check(self.hip.hipEventRecord(self.ev[i], ctypes.c_void_p(stream)), "hipEventRecord")

    def elapsed_ms(self):
        ms = ctypes.c_float()
        self._check(self.hip.hipEventElapsedTime(ctypes.byref(ms), self.ev[0], self.ev[1]), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        for e in getattr(self, "ev", []):
            if e:
                self.hip.hipEventDestroy(e)


_EVENTS = None


def _replay_timed(torch, graph, n, reps=1):
    """Replay a captured graph of n launches: one untimed warm replay (the
    first replay of a graph also uploads it), then `reps` timed replays, each
    between synchronisations with HIP timing events (no system-scope fence) on
    the launch stream.  Returns the ms per launch of every timed replay (the
    first one is the headline)."""
    global _EVENTS
    if _EVENTS is None:
        _EVENTS = _TimingEvents()
    graph.replay()
    torch.cuda.synchronize()
    out = []
    for _ in range(reps):
        stream = torch.cuda.current_stream().cuda_stream
        _queue_ahead(torch)
        _EVENTS.record(0, stream)
        graph.replay()
        _EVENTS.record(1, stream)
        torch.cuda.synchronize()
        out.append(_EVENTS.elapsed_ms() / n)
    return out if reps > 1 else out[0]


def _median_timed(torch, graph, n, reps=5):
    """Median ms per launch over `reps` timed replays (after the warm one):
    the first replays after a change of kernel can run at a lower clock."""
    return float(np.median(_replay_timed(torch, graph, n, reps)))


def run_decode(T, R, steps, warmup, seed, bits=8, kind="outliers", frac=0.01, batch=1, reps=5, hq=HQ, hkv=HKV):
    import torch

    total = warmup + 2 * steps
    log(f"T={T}: building {R} cache instances")
    w = DecodeWorkload(T, R, total, seed, bits=bits, kind=kind, frac=frac, batch=batch, hq=hq, hkv=hkv)
    log(f"T={T}: warm-up {warmup} steps")
    for s in range(warmup):
        w.step(s)
    torch.cuda.synchronize()
    # K whole steps (attention kernel + merge kernel) in one graph.  A replay
    # rewrites the appended tokens at the same positions with the same values,
    # so every replay does the same work: one untimed warm replay, then `reps`
    # timed replays of exactly K steps each; the headline is their median,
    # p10/p50/p90 their spread.
    g_step, step_T = torch.cuda.CUDAGraph(), []
    with torch.cuda.graph(g_step):
        for s in range(warmup, warmup + steps):
            step_T.append(w.step(s))
    # K launches of the attention kernel alone, the dominant kernel
    g_kern, kern_T = torch.cuda.CUDAGraph(), []
    with torch.cuda.graph(g_kern):
        for s in range(warmup + steps, total):
            kern_T.append(w.step(s, partial_only=True))
    # the unfused halves of a step, each K times: attention over the cached
    # tokens (two launches) and the append of one token (one launch)
    g_att, g_app = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_att):
        for s in range(steps):
            w.attend_only(s)
    with torch.cuda.graph(g_app):
        for s in range(steps):
            w.append_only(s)
    rep_ms = _replay_timed(torch, g_step, steps, reps)
    ms_per_step = float(np.median(rep_ms))
    kernel_ms = _median_timed(torch, g_kern, steps)
    att_ms = _median_timed(torch, g_att, steps)
    app_ms = _median_timed(torch, g_app, steps)
    p10, p50, p90 = (float(np.percentile(rep_ms, p)) for p in (10, 50, 90))
    log(f"T={T}: {steps} steps, {ms_per_step * 1e3:.2f} us/step (replays p10/p50/p90 {p10 * 1e3:.2f}/"
        f"{p50 * 1e3:.2f}/{p90 * 1e3:.2f}); attention kernel {kernel_ms * 1e3:.2f} us; unfused: attention "
        f"{att_ms * 1e3:.2f} us + append {app_ms * 1e3:.2f} us")
    bytes_step = float(np.mean([step_bytes(t, batch, k_bits=bits, v_bits=bits, hq=hq, hkv=hkv) for t in step_T]))
    bytes_kernel = float(np.mean([step_bytes(t, batch, k_bits=bits, v_bits=bits, output=False, hq=hq, hkv=hkv)
                                  for t in kern_T]))
    res = dict(
        T=T,
        instances=R,
        ms_per_step=ms_per_step,
        us_per_step=ms_per_step * 1e3,
        bytes_per_step=bytes_step,
        gbs=bytes_step / (ms_per_step * 1e-3) / 1e9,
        kernel_us=kernel_ms * 1e3,
        kernel_gbs=bytes_kernel / (kernel_ms * 1e-3) / 1e9,
        bytes_per_launch=bytes_kernel,
        cache_bytes=sum(c.nbytes for c in w.caches),
        step_us_p10_p50_p90=[round(p10 * 1e3, 3), round(p50 * 1e3, 3), round(p90 * 1e3, 3)],
        unfused_attention_us=att_ms * 1e3,
        unfused_append_us=app_ms * 1e3,
    )
    del g_step, g_kern, g_att, g_app, w
    torch.cuda.empty_cache()
    return res


def bf16_step_bytes(T, B=1):
    """Algorithmic HBM bytes of one bf16-cache decode step: K/V rows of T tokens
    (2 x 256 B per token and head), query, fp32 output, new token read + written."""
    return B * (T * HKV * 2 * D * 2 + HQ * D * 2 + HQ * D * 4 + 2 * HKV * 2 * D * 2)


def run_decode_bf16(T, R, steps, warmup, seed):
    """Decode steps over the reference's production bf16 cache (KVStorage /
    FixedKVCache): fused write of the new token + attention + merge, rotating
    R single-layer storages."""
    import torch

    import rec_amd
    from rec_amd import synthetic
    from rec_amd.attention import _bf16_decode_launch

    log(f"bf16 T={T}: building {R} storages")
    caches = []
    for i in range(R):
        c = rec_amd.FixedKVCache(rec_amd.KVStorage(1, T, HKV), 0)
        k = synthetic.kv((1, HKV, T - 1, D), seed + 2 * i, kind="outliers", frac=0.01, dtype=torch.bfloat16)
        v = synthetic.kv((1, HKV, T - 1, D), seed + 2 * i + 1, kind="outliers", frac=0.01, dtype=torch.bfloat16)
        c.update_and_fetch(k, v)
        del k, v
        caches.append(c)
    q = synthetic.query(1, HQ, 1, seed + 100, dtype=torch.bfloat16)
    kn = synthetic.kv((1, HKV, 1, D), seed + 101, dtype=torch.bfloat16)
    vn = synthetic.kv((1, HKV, 1, D), seed + 102, dtype=torch.bfloat16)
    g0 = torch.Generator(device="cuda")
    g0.manual_seed(seed)
    sinks = torch.randn(HQ, generator=g0, device="cuda")
    out = torch.empty((1, HQ, D), dtype=torch.float32, device="cuda")

    def step(s):
        c = caches[s % R]
        data = c.storage.layer(0)
        _bf16_decode_launch(q, data[:, 0], data[:, 1], SCALE, sinks, None, out, kn, vn, T=T,
                            capacity=c.storage.capacity)

    for s in range(warmup):
        step(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for s in range(steps):
            step(s)
    ms = _median_timed(torch, g, steps)
    gbs = bf16_step_bytes(T) / (ms * 1e-3) / 1e9
    log(f"bf16 T={T}: {ms * 1e3:.2f} us/step, {gbs:.0f} GB/s")
    res = dict(
        context=T,
        kv_format="bf16 token-major [2][Hkv][cap][128] (KVStorage)",
        us_per_step=round(ms * 1e3, 3),
        gbs=round(gbs, 2),
        frac_of_peak=round(gbs / HBM_PEAK_GBS, 4),
        bytes_per_step=bf16_step_bytes(T),
        storages=R,
        note="fused write of the new token + attention + merge per step",
    )
    del g, caches
    torch.cuda.empty_cache()
    return res


# (rows N, features K, name) of the int4 projections of one decode token
Q4_SHAPES = [
    (150144, 2048, "lm_head"),
    (6144, 2048, "dense_gate_up"),
    (2048, 6144, "dense_down"),
    (4096, 2048, "q_proj"),
    (2048, 4096, "o_proj"),
    (512, 2048, "k_proj"),
    (5120, 2048, "qkv_proj"),  # q, k and v stacked (Q4Matrix.stack): one launch for the three
]


def run_q4_gemm(steps, seed, M=2048):
    """The int4 matrix for a prefill chunk's M tokens (rec_q4_gemm: the same
    packed matrix as the GEMV, one GEMM), at the q projection and the dense
    gate/up shapes; beside it PyTorch's bf16 matmul over an already
    dequantized matrix of the same shape (the library's GEMM, a yardstick:
    4x the weight bytes and no dequantization)."""
    import torch

    import rec_amd

    res = {}
    for N, K, name in ((4096, 2048, "q_proj"), (6144, 2048, "dense_gate_up")):
        g = torch.Generator(device="cuda")
        g.manual_seed(seed + N)
        w = torch.randint(-(2**31), 2**31 - 1, (N, K // 8), dtype=torch.int32, device="cuda", generator=g)
        s = (torch.rand((N, K // 64), device="cuda", generator=g) * 0.05).to(torch.bfloat16)
        b = (torch.rand((N, K // 64), device="cuda", generator=g) * 0.1).to(torch.bfloat16)
        m = rec_amd.Q4Matrix(w, s, b)
        x = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
        out = torch.empty((M, N), device="cuda", dtype=torch.bfloat16)
        dense = torch.randn((N, K), device="cuda", generator=g).to(torch.bfloat16)
        times = {}
        for what, fn in (("q4", lambda: out.copy_(rec_amd.q4_gemv(x, m))), ("bf16", lambda: torch.matmul(x, dense.T))):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                for _ in range(steps):
                    fn()
            times[what] = _median_timed(torch, gr, steps)
            del gr
        fl = 2.0 * M * N * K
        tf = fl / (times["q4"] * 1e-3) / 1e12
        log(f"q4 gemm {name} {M}x{N}x{K}: {times['q4'] * 1e3:.1f} us, {tf:.0f} TFLOP/s "
            f"(bf16 matmul over dense weights {times['bf16'] * 1e3:.1f} us)")
        res[name] = dict(M=M, N=N, K=K, us=round(times["q4"] * 1e3, 2), tflops=round(tf, 1),
                         frac_of_mfma_peak=round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                         library_yardstick=dict(us=round(times["bf16"] * 1e3, 2),
                                                what="torch.matmul over a dense bf16 matrix of the same shape"))
        del m, w, s, b, dense
        torch.cuda.empty_cache()
    return res


def run_q4_gemv(steps, seed):
    """int4 group-64 GEMV (one bf16 vector) at the decoder's projection
    shapes; each launch reads a different copy of the packed matrix (about
    600 MB of copies in rotation) so no launch finds its weights in cache."""
    import torch

    import rec_amd
    from rec_amd import _lib

    lib = rec_amd.library()
    res = {}
    for N, K, name in Q4_SHAPES:
        g = torch.Generator(device="cuda")
        g.manual_seed(seed + N + K)
        w = torch.randint(-(2**31), 2**31 - 1, (N, K // 8), dtype=torch.int32, device="cuda", generator=g)
        s = (torch.rand((N, K // 64), device="cuda", generator=g) * 0.05).to(torch.bfloat16)
        b = (torch.rand((N, K // 64), device="cuda", generator=g) * 0.1).to(torch.bfloat16)
        base = rec_amd.Q4Matrix(w, s, b)
        del w, s, b
        nb = base.nbytes
        copies = max(2, -(-600_000_000 // nb))
        packs = [base.packed] + [base.packed.clone() for _ in range(copies - 1)]
        x = torch.randn((1, K), device="cuda", generator=g).to(torch.bfloat16)
        out = torch.empty((1, N), device="cuda", dtype=torch.bfloat16)

        def step(i):
            rc = lib.rec_q4_gemv(packs[i % copies].data_ptr(), N, K, x.data_ptr(), K, 1, out.data_ptr(),
                                 _lib.REC_BF16, N, torch.cuda.current_stream().cuda_stream)
            _lib.check(rc, "q4 gemv")

        n = steps if nb > 50e6 else 4 * steps
        for i in range(4):
            step(i)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for i in range(n):
                step(i)
        ms = _median_timed(torch, gr, n)
        byts = nb + 2 * K + 2 * N
        gbs = byts / (ms * 1e-3) / 1e9
        log(f"q4 gemv {name} {N}x{K}: {ms * 1e3:.2f} us, {gbs:.0f} GB/s")
        res[name] = dict(N=N, K=K, us=round(ms * 1e3, 3), gbs=round(gbs, 2), frac_of_peak=round(gbs / HBM_PEAK_GBS, 4),
                         bytes_per_launch=byts, copies=copies)
        del gr, packs, base
        torch.cuda.empty_cache()
    return res


MFMA_BF16_PEAK_TFLOPS = 2500.0


PREFILL_FORMATS = {
    "int8": "int8 symmetric, fp16 scale per (token, head)",
    "uint4": "uint4 asymmetric, fp16 scale + zero-point per 32 dims",
    "affine": "MLX-style affine group 64: 8-bit K, 4-bit V, bf16 scale + bias",
    "bf16": "bf16 token-major (KVStorage / FixedKVCache, the reference's production cache)",
}


def run_prefill(P, L, steps, warmup, seed, fmt="int8"):
    """Chunked prefill: append L new tokens after a P-token prefix in the
    cache format `fmt` (quantized, or written as bf16 into a KVStorage), then
    L causal bf16 queries attend over all P + L tokens, every K/V tile
    dequantized (or converted) on chip.  Each step rewrites the same L
    positions, so every step does identical work."""
    import torch

    import rec_amd
    from rec_amd import _lib, synthetic

    lib = rec_amd.library()
    T = P + L
    log(f"prefill ({fmt}): building a {P}-token prefix")
    bf = fmt == "bf16"
    if bf:
        c = rec_amd.FixedKVCache(rec_amd.KVStorage(1, T, HKV), 0)
    elif fmt == "affine":
        c = rec_amd.MixedQuantizedKVCache(max_tokens=T)
    else:
        bits = 8 if fmt == "int8" else 4
        c = rec_amd.QuantizedKVCache(32, bits, bits, max_tokens=T)
    kdt = torch.bfloat16 if bf or fmt == "affine" else torch.float16  # affine: a bf16 model's cache
    k = synthetic.kv((1, HKV, P, D), seed, kind="outliers", frac=0.01, dtype=kdt)
    v = synthetic.kv((1, HKV, P, D), seed + 1, kind="outliers", frac=0.01, dtype=kdt)
    c.update_and_fetch(k, v)
    del k, v
    kn = synthetic.kv((1, HKV, L, D), seed + 2, kind="outliers", frac=0.01, dtype=torch.bfloat16)
    vn = synthetic.kv((1, HKV, L, D), seed + 3, kind="outliers", frac=0.01, dtype=torch.bfloat16)
    q = synthetic.query(1, HQ, L, seed + 4, dtype=torch.bfloat16)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    sinks = torch.randn(HQ, generator=g, device="cuda")
    out = torch.empty((1, HQ, L, D), dtype=torch.float32, device="cuda")
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    if bf:
        data = c.storage.layer(0)
        kr, vr = data[:, 0], data[:, 1]
        tok_bytes = 2 * D * 2  # bf16 K and V rows
    else:
        c._reserve(1, HKV, T, "cuda")
        kq, vq = c.keys_and_values()
        # cache bytes per (token, kv head): codes + scales (+ zero-points) of K and V
        tok_bytes = sum(t.nbytes for kv in (kq, vq) for t in (kv.codes, kv.scales, kv.zeros) if t is not None)
        tok_bytes /= HKV * c.capacity
    # key splits when the chunk is short (the automatic plan; none at 2048 queries)
    ws = torch.empty(max(16, lib.rec_prefill_workspace_bytes(1, HQ, HKV, L, 0)), dtype=torch.uint8, device="cuda")

    def append():
        st = torch.cuda.current_stream().cuda_stream
        if bf:
            rc = lib.rec_kv_write_bf16(kn.data_ptr(), vn.data_ptr(), _lib.REC_BF16, *kn.stride()[:3], *vn.stride()[:3],
                                       kr.data_ptr(), kr.stride(0), kr.stride(1), vr.data_ptr(), vr.stride(0),
                                       vr.stride(1), 1, HKV, L, D, P, c.storage.capacity, st)
            _lib.check(rc, "rec_kv_write_bf16")
            return
        rc = lib.rec_kv_append(kn.data_ptr(), vn.data_ptr(), _lib.REC_BF16, *kn.stride()[:3], *vn.stride()[:3],
                               kq.code, kq.codes.data_ptr(), kq.scales.data_ptr(), ptr(kq.zeros),
                               vq.code, vq.codes.data_ptr(), vq.scales.data_ptr(), ptr(vq.zeros),
                               1, HKV, L, D, P, c.capacity, st)
        _lib.check(rc, "rec_kv_append")

    def attention():
        st = torch.cuda.current_stream().cuda_stream
        if bf:
            rc = lib.rec_prefill_bf16(q.data_ptr(), _lib.REC_BF16, *q.stride()[:3], kr.data_ptr(), kr.stride(0),
                                      kr.stride(1), vr.data_ptr(), vr.stride(0), vr.stride(1), sinks.data_ptr(), SCALE,
                                      1, 0, None, 0, 0, 0, 0, 0, 1, HQ, HKV, D, L, T, 0, ws.data_ptr(), ws.numel(),
                                      _lib.REC_F32,
                                      out.data_ptr(), st)
            _lib.check(rc, "rec_prefill_bf16")
            return
        rc = lib.rec_prefill_attn(q.data_ptr(), _lib.REC_BF16, *q.stride()[:3],
                                  kq.code, kq.codes.data_ptr(), kq.scales.data_ptr(), ptr(kq.zeros),
                                  vq.code, vq.codes.data_ptr(), vq.scales.data_ptr(), ptr(vq.zeros),
                                  sinks.data_ptr(), SCALE, 1, 0, None, 0, 0, 0, 0, 0,
                                  1, HQ, HKV, D, L, T, c.capacity, 0, ws.data_ptr(), ws.numel(), _lib.REC_F32,
                                  out.data_ptr(), st)
        _lib.check(rc, "rec_prefill_attn")

    for _ in range(warmup):
        append()
        attention()
    torch.cuda.synchronize()
    g_step, g_att, g_app = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_step):
        for _ in range(steps):
            append()
            attention()
    with torch.cuda.graph(g_att):
        for _ in range(steps):
            attention()
    with torch.cuda.graph(g_app):
        for _ in range(steps):
            append()
    ms_step = _median_timed(torch, g_step, steps)
    ms_att = _median_timed(torch, g_att, steps)
    ms_app = _median_timed(torch, g_app, steps)
    pairs = L * P + L * (L + 1) // 2
    flops = 4.0 * D * HQ * pairs
    tflops = flops / (ms_att * 1e-3) / 1e12
    kv_bytes = round(T * HKV * tok_bytes)  # every cached K/V row and its scales, read once
    log(f"prefill ({fmt}) {P}+{L}: {ms_step:.3f} ms/step, attention {ms_att:.3f} ms = {tflops:.0f} TFLOP/s, "
        f"{kv_bytes / (ms_att * 1e-3) / 1e9:.0f} GB/s of K/V")
    del g_step, g_att, g_app, c
    torch.cuda.empty_cache()
    return dict(
        prefix=P,
        new_tokens=L,
        kv_format=PREFILL_FORMATS[fmt],
        ms_per_step=round(ms_step, 4),
        append_ms=round(ms_app, 4),
        attention_ms=round(ms_att, 4),
        attention_flops=flops,
        attention_tflops=round(tflops, 1),
        frac_of_mfma_peak=round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
        mfma_peak_tflops=MFMA_BF16_PEAK_TFLOPS,
        kv_bytes=kv_bytes,
        kv_gbs=round(kv_bytes / (ms_att * 1e-3) / 1e9, 2),
        kv_frac_of_hbm_peak=round(kv_bytes / (ms_att * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        note="Q.K^T on bf16 MFMA, P.V on fp16 MFMA; peak is the dense bf16 figure",
    )


def run_sliding(steps, seed, window=513, held=4096, chunk=512):
    """A sliding-window layer (FixedSlidingKVCache, the reference's 513-token
    window, bf16 ring): one decode step (token written into its ring slot,
    attention over the window) and one 512-token chunk (written into the ring,
    attending over the window in order plus itself under the causal window
    mask), each through attend() in a graph of `steps` calls.  Every replay
    writes the same slots, so every call does identical work."""
    import torch

    import rec_amd
    from rec_amd import synthetic

    c = rec_amd.FixedSlidingKVCache(max_sequence_tokens=held + 2 * chunk, num_kv_heads=HKV, head_dim=D,
                                    window_size=window)
    k = synthetic.kv((1, HKV, held, D), seed, dtype=torch.bfloat16)
    v = synthetic.kv((1, HKV, held, D), seed + 1, dtype=torch.bfloat16)
    for a in range(0, held, chunk):
        c.update_and_fetch(k[:, :, a:a + chunk], v[:, :, a:a + chunk])
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    sinks = torch.randn(HQ, generator=g, device="cuda")
    q1 = synthetic.query(1, HQ, 1, seed + 2, dtype=torch.bfloat16)
    k1 = synthetic.kv((1, HKV, 1, D), seed + 3, dtype=torch.bfloat16)
    v1 = synthetic.kv((1, HKV, 1, D), seed + 4, dtype=torch.bfloat16)
    qc = synthetic.query(1, HQ, chunk, seed + 5, dtype=torch.bfloat16)
    kc = synthetic.kv((1, HKV, chunk, D), seed + 6, dtype=torch.bfloat16)
    vc = synthetic.kv((1, HKV, chunk, D), seed + 7, dtype=torch.bfloat16)
    out = {}
    # the library keeps one workspace per stream: a first call on the capture
    # stream, outside the capture, allocates it there, so the graph reuses it
    cap_stream = torch.cuda.Stream()
    for name, (q, kk, vv) in (("decode", (q1, k1, v1)), ("chunk", (qc, kc, vc))):
        call = lambda: rec_amd.attend(q, kk, vv, c, SCALE, None, sinks)  # noqa: E731
        cap_stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cap_stream):
            call()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=cap_stream):
            for _ in range(steps):
                call()
        out[name] = _median_timed(torch, graph, steps) * 1e3
        del graph
    log(f"sliding window {window}: decode step {out['decode']:.2f} us, {chunk}-token chunk {out['chunk']:.2f} us")
    return dict(
        window=window,
        decode_step_us=round(out["decode"], 3),
        chunk_tokens=chunk,
        chunk_us=round(out["chunk"], 3),
        note="FixedSlidingKVCache (bf16 ring, 513-token window as the reference's sliding layers), through "
             "attend(): decode = token written into its slot by the attention launch + merge; chunk = 512 tokens written "
             "into the ring, then attention over the window in order plus the chunk under the causal window mask; "
             "both latency-bound (the window is 513 tokens)",
    )


def run_sdpa_yardstick(P, L, steps):
    """A library yardstick for the prefill, not this library's kernel: PyTorch's
    own fused attention (torch.nn.functional.scaled_dot_product_attention,
    flash backend, bf16 K/V already in HBM with the KV heads expanded to the
    query heads, causal aligned to the last query) over the same P + L keys,
    timed on the current stream over `steps` back-to-back calls."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from torch.nn.attention.bias import causal_lower_right

    T = P + L
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    q = torch.randn(1, HQ, L, D, device="cuda", dtype=torch.bfloat16, generator=g)
    k = torch.randn(1, HQ, T, D, device="cuda", dtype=torch.bfloat16, generator=g)
    v = torch.randn(1, HQ, T, D, device="cuda", dtype=torch.bfloat16, generator=g)
    mask = causal_lower_right(L, T)
    try:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            call = lambda: F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=float(SCALE))  # noqa: E731
            call()
            torch.cuda.synchronize()
            times = []
            for _ in range(5):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                for _ in range(steps):
                    call()
                b.record()
                torch.cuda.synchronize()
                times.append(a.elapsed_time(b) / steps)
    except Exception as e:  # no fused kernel for this device or shape
        log(f"sdpa yardstick unavailable: {e}")
        return None
    finally:
        del q, k, v
        torch.cuda.empty_cache()
    ms = sorted(times)[2]
    flops = 4.0 * D * HQ * (L * P + L * (L + 1) // 2)
    log(f"sdpa yardstick {P}+{L}: {ms:.3f} ms = {flops / (ms * 1e-3) / 1e12:.0f} TFLOP/s")
    return dict(
        ms=round(ms, 4),
        tflops=round(flops / (ms * 1e-3) / 1e12, 1),
        what="torch.nn.functional.scaled_dot_product_attention (flash backend) over the same causal chunk, bf16 K/V "
             "expanded to 32 heads, no quantization and no sinks; PyTorch's own kernel, not this library's",
    )


def run_read_floor(steps):
    """The one-launch read floor of this part: rec_stream_read (a plain
    streaming read, 1 KB per wavefront and load, four loads in flight per
    lane) over the K/V bytes of the 32K and 252K int8 configurations and the
    131K uint4 one, rotating buffers of >= 1 GB in all; the best of five
    workgroup counts."""
    import torch

    import rec_amd

    lib = rec_amd.library()
    out = torch.zeros(65536, dtype=torch.int32, device="cuda")
    res = {}
    for name, T, R, n, bits in (("32k", 32768, 32, steps, 8), ("252k", 258048, 4, max(16, steps // 8), 8),
                                ("131k_int4", 131072, 12, max(16, steps // 8), 4)):
        nbytes = T * HKV * (row_bytes(bits) + row_bytes(bits, True))
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(i + 1) for i in range(R)]
        best = None
        for wg in (256, 512, 1024, 2048, 4096):
            def launch(i, wg=wg):
                rc = lib.rec_stream_read(bufs[i % R].data_ptr(), nbytes, wg, out.data_ptr(),
                                         torch.cuda.current_stream().cuda_stream)
                assert rc == 0, rc
            launch(0)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(n):
                    launch(i)
            us = _median_timed(torch, g, n) * 1e3
            log(f"read floor {name}: {wg} workgroups {us:.2f} us")
            if best is None or us < best[0]:
                best = (us, wg)
            del g
        us, wg = best
        gbs = nbytes / (us * 1e-6) / 1e9
        log(f"read floor {name}: {nbytes} B in {us:.2f} us = {gbs:.0f} GB/s ({wg} workgroups)")
        res[name] = dict(bytes=nbytes, us=round(us, 3), gbs=round(gbs, 1), frac_of_peak=round(gbs / HBM_PEAK_GBS, 4),
                         workgroups=wg)
        del bufs
        torch.cuda.empty_cache()
    return res


def host_cores():
    """Host cores this process may run on (its CPU affinity), bounded by the
    thread budget OMP_NUM_THREADS when the environment sets one (a shared GPU
    host gives each GPU's jobs a share of its cores that way)."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, n)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(T, seed, budget_s=10.0, bits=8, hq=HQ, hkv=HKV, kind="outliers", frac=0.01, label="32K"):
    """The oracle's split-K decode over one cache instance of the configuration
    on the host cores: each step quantizes the new token (the oracle's
    quantizer) into the last slot and runs the float32 split-K over 4096-token
    chunks (chunked dequantization, attention with sinks, merge)."""
    import torch

    import oracle as O
    import rec_amd
    from rec_amd import synthetic

    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    cores = host_cores()
    c = rec_amd.QuantizedKVCache(32, bits, bits, max_tokens=T)
    k = synthetic.kv((1, hkv, T - 1, D), seed, kind=kind, frac=frac)
    v = synthetic.kv((1, hkv, T - 1, D), seed + 1, kind=kind, frac=frac)
    kq, vq = c.update_and_fetch(k, v)
    logical = [[None if x is None else x.cpu().numpy() for x in rec_amd.to_logical(t)] for t in (kq, vq)]
    del k, v, c, kq, vq
    torch.cuda.empty_cache()
    bufs = {}
    for p, (codes, scales, zeros) in zip("kv", logical):
        for name, a in (("q", codes), ("s", scales), ("z", zeros)):
            if a is None:
                continue
            full = np.zeros(a.shape[:2] + (T,) + a.shape[3:], a.dtype)
            full[:, :, : T - 1] = a
            bufs[p + name] = full
    del logical
    quant = O.quantize_int8 if bits == 8 else (lambda x: O.quantize_int4(x, 32))
    rng = np.random.default_rng(seed)
    sinks = rng.standard_normal(hq).astype(np.float32)
    times = []
    limiter = threadpool_limits(1) if threadpool_limits else None
    try:
        start = time.perf_counter()
        while True:
            q = rng.standard_normal((1, hq, D)).astype(np.float16).astype(np.float32)
            kn = rng.standard_normal((1, hkv, 1, D)).astype(np.float16)
            vn = rng.standard_normal((1, hkv, 1, D)).astype(np.float16)
            t0 = time.perf_counter()
            for p, x in (("k", kn), ("v", vn)):
                for name, a in zip("qsz", quant(x)):
                    bufs[p + name][:, :, T - 1 :] = a
            cache = dict(k_bits=bits, v_bits=bits, **bufs)
            O.split_k_decode_quantized(q, cache, T, SCALE, sinks, chunk=4096, workers=cores)
            times.append(time.perf_counter() - t0)
            if time.perf_counter() - start > budget_s and len(times) >= 3:
                break
    finally:
        if limiter is not None:
            limiter.unregister()
    sec = float(np.median(times))
    fmt = "int8" if bits == 8 else "uint4"
    return dict(
        value=step_bytes(T, k_bits=bits, v_bits=bits, hq=hq, hkv=hkv) / sec / 1e9,
        unit="GB/s",
        cores=cores,
        affinity_cores=len(os.sched_getaffinity(0)),
        cpu_model=cpu_model(),
        kind="port",
        us_per_step=sec * 1e6,
        sample=f"{len(times)} decode steps (1-token {fmt} append + attention) of the {label} workload "
        f"({hq} q / {hkv} kv heads, {T} tokens), one cache instance, NumPy float32 split-K over 4096-token "
        f"chunks on {cores} threads; median step time",
    )


def _step_detail(r):
    """Spread of the fused step over the timed replays, and the two halves
    of an unfused step timed alone (attention = partial + merge launches;
    append = one rec_kv_append launch)."""
    return {
        "us_per_step_p10_p50_p90": r["step_us_p10_p50_p90"],
        "unfused_attention_us": round(r["unfused_attention_us"], 3),
        "unfused_append_us": round(r["unfused_append_us"], 3),
    }


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--long-steps", type=int, default=0, help="timed steps at 252K (default steps/8)")
    ap.add_argument("--no-long", action="store_true", help="skip the 252K measurement")
    ap.add_argument("--no-prefill", action="store_true", help="skip the chunked-prefill measurement")
    ap.add_argument("--no-int4", action="store_true", help="skip the 131K uint4 measurement")
    ap.add_argument("--no-batch", action="store_true", help="skip the 32K batch-4 measurement")
    ap.add_argument("--no-bf16", action="store_true", help="skip the bf16-cache measurements")
    ap.add_argument("--no-gemv", action="store_true", help="skip the int4 GEMV measurements")
    ap.add_argument("--no-affine", action="store_true", help="skip the group-64 affine cache measurement")
    ap.add_argument("--prefill-steps", type=int, default=6)
    ap.add_argument("--no-floor", action="store_true", help="skip the plain streaming-read floor")
    ap.add_argument("--no-yardstick", action="store_true", help="skip timing PyTorch's own fused attention")
    ap.add_argument("--no-sliding", action="store_true", help="skip the sliding-window layer measurement")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-tiny", action="store_true", help="skip the 1,024-token 8:1 configuration")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument(
        "--calibrate",
        action="store_true",
        help="first run two plain 256 MiB device copies (a known-size kernel for hardware-counter scaling)",
    )
    args = ap.parse_args(argv)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
            "the decode path shards by KV head or by context with no per-step collective beyond a "
            "16.6 KB merge, which this single-GPU build does not run",
            file=sys.stderr,
        )
        return 2

    import torch

    import rec_amd

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    rec_amd.library()
    torch.cuda.set_device(0)
    if args.calibrate:
        src = torch.ones(CALIB_BYTES, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(2):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        log(f"calibration: 2 copies of {CALIB_BYTES} bytes")

    r32 = run_decode(32768, 32, args.steps, args.warmup, args.seed)
    log(f"32K: {r32['us_per_step']:.2f} us/step, {r32['gbs']:.0f} GB/s; kernel {r32['kernel_us']:.2f} us")
    r1k = None
    if not args.no_tiny:
        # the CPU-sized parity configuration: 8 q heads over 1 KV head, 1,024
        # tokens, N(0, 1) K/V; 64 instances (17 MB) stay in the MALL, so this
        # is a launch-latency figure
        r1k = run_decode(1024, 64, max(16, args.steps // 4), max(4, args.warmup // 4), args.seed + 11, kind="normal",
                         frac=0.0, hq=8, hkv=1)
        log(f"1K tiny: {r1k['us_per_step']:.2f} us/step; kernel {r1k['kernel_us']:.2f} us")
    r252 = None
    if not args.no_long:
        ls = args.long_steps or max(16, args.steps // 8)
        r252 = run_decode(258048, 4, ls, max(4, args.warmup // 4), args.seed + 99)
        log(f"252K: {r252['us_per_step']:.2f} us/step, {r252['gbs']:.0f} GB/s; kernel {r252['kernel_us']:.2f} us")

    rb4 = None
    if not args.no_batch:
        # the 32K configuration for 4 sequences at once: the same two launches
        # per step carry 4x the bytes, which separates the fixed per-step cost
        # (launches, first-load latency) from the kernel's streaming rate
        rb4 = run_decode(32768, 8, max(16, args.steps // 4), max(4, args.warmup // 4), args.seed + 55, batch=4)
        log(f"32K batch 4: {rb4['us_per_step']:.2f} us/step, {rb4['gbs']:.0f} GB/s; kernel {rb4['kernel_us']:.2f} us")

    r4 = None
    if not args.no_int4:
        ls = args.long_steps or max(16, args.steps // 8)
        r4 = run_decode(131072, 12, ls, max(4, args.warmup // 4), args.seed + 77, bits=4, kind="heavy", frac=0.05)
        log(f"131K int4: {r4['us_per_step']:.2f} us/step, {r4['gbs']:.0f} GB/s; kernel {r4['kernel_us']:.2f} us")

    raf = raf252 = None
    if not args.no_affine:
        raf = run_decode(32768, 40, max(16, args.steps // 4), max(4, args.warmup // 4), args.seed + 88, bits=AFFINE)
        log(f"32K affine: {raf['us_per_step']:.2f} us/step, {raf['gbs']:.0f} GB/s; kernel {raf['kernel_us']:.2f} us")
        if not args.no_long:
            ls = args.long_steps or max(16, args.steps // 8)
            raf252 = run_decode(258048, 5, ls, max(4, args.warmup // 4), args.seed + 89, bits=AFFINE)
            log(f"252K affine: {raf252['us_per_step']:.2f} us/step, {raf252['gbs']:.0f} GB/s; "
                f"kernel {raf252['kernel_us']:.2f} us")

    rbf = {}
    if not args.no_bf16:
        ls = args.long_steps or max(16, args.steps // 8)
        rbf["context_32k_bf16"] = run_decode_bf16(32768, 8, max(16, args.steps // 4), 8, args.seed + 61)
        rbf["context_252k_bf16"] = run_decode_bf16(258048, 2, ls, 4, args.seed + 63)

    rq4 = None
    if not args.no_gemv:
        rq4 = run_q4_gemv(max(16, args.steps // 16), args.seed + 41)
        rq4m = run_q4_gemm(10, args.seed + 43)

    rpf = rpf_short = rpf_short_u4 = rpf_few = rpf_few_affine = rpf_few_u4 = None
    rpf_fmt = {}
    if not args.no_prefill:
        rpf = run_prefill(65536, 2048, args.prefill_steps, 2, args.seed + 51)
        # a short chunk over a long cache (a new chat turn), the keys split: 160
        # (query, head) rows per KV head stream in row groups over the int8
        # cache; the uint4 one keeps the tiled kernel
        rpf_short = run_prefill(32768, 20, max(10, args.steps // 20), 2, args.seed + 53)
        rpf_short_u4 = run_prefill(32768, 20, max(10, args.steps // 20), 2, args.seed + 56, "uint4")
        # four draft tokens over a long cache: the streaming few-query kernel
        rpf_few = run_prefill(65536, 4, max(10, args.steps // 20), 2, args.seed + 54)
        rpf_few_affine = run_prefill(65536, 4, max(10, args.steps // 20), 2, args.seed + 54, "affine")
        rpf_few_u4 = run_prefill(65536, 4, max(10, args.steps // 20), 2, args.seed + 57, "uint4")
        # the same long chunk over the 4-bit, affine and bf16 caches
        for i, fmt in enumerate(("uint4", "affine", "bf16")):
            rpf_fmt[fmt] = run_prefill(65536, 2048, args.prefill_steps, 2, args.seed + 55 + 2 * i, fmt)
        if not args.no_yardstick:
            rpf["library_yardstick"] = run_sdpa_yardstick(65536, 2048, args.prefill_steps)

    sliding = None
    if not args.no_bf16 and not args.no_sliding:
        try:
            sliding = run_sliding(max(10, args.steps // 20), args.seed + 61)
        except Exception as e:  # a measurement beside the headline; the line is printed without it
            log(f"sliding-window measurement failed: {e}")

    floor = None if args.no_floor else run_read_floor(max(20, args.steps // 5))

    traffic, traffic_source, traffic_cfg = None, None, {}
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        traffic_cfg = t.get("configs", {})
        traffic = traffic_cfg.get("32k_int8", {}).get("hbm_bytes_per_launch")
        traffic_source = (f"not measured by this run: {os.path.relpath(TRAFFIC_FILE, ROOT)}, rocprofv3 FETCH_SIZE and "
                          f"WRITE_SIZE passes over this kernel at source commit {t.get('source_commit', 'unrecorded')}")

    def traffic_of(name):
        c = traffic_cfg.get(name)
        return None if c is None else dict(hbm_bytes_per_launch=c["hbm_bytes_per_launch"], ratio_to_algorithmic=c["ratio"],
                                           source=traffic_source)

    cpu = None
    cpu_more = {}
    if not args.no_cpu_baseline:
        log("CPU baseline")
        cpu = cpu_baseline(32768, args.seed + 7, args.cpu_budget)
        # the other decode configurations, each beside its GPU figure
        b = max(3.0, 0.6 * args.cpu_budget)
        if r1k is not None:
            cpu_more["context_1k_tiny"] = cpu_baseline(1024, args.seed + 8, b, hq=8, hkv=1, kind="normal", frac=0.0,
                                                       label="1K 8:1")
        if r252 is not None:
            cpu_more["context_252k"] = cpu_baseline(258048, args.seed + 9, b, label="252K")
        if r4 is not None:
            cpu_more["context_131k_int4"] = cpu_baseline(131072, args.seed + 10, b, bits=4, kind="heavy", frac=0.05,
                                                         label="131K uint4")
        for name, c in cpu_more.items():
            log(f"CPU baseline {name}: {c['us_per_step']:.0f} us/step, {c['value']:.1f} GB/s on {c['cores']} threads")

    result = {
        "metric": METRIC,
        "value": round(r32["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r32["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": "decode step at 32K context: 1-token int8 quantize-append + GQA attention, 32 q heads / "
            "4 kv heads, head_dim 128, batch 1, one layer",
            "context": 32768,
            "q_heads": HQ,
            "kv_heads": HKV,
            "head_dim": D,
            "batch": 1,
            "kv_format": "int8 symmetric, fp16 scale per (token, head); 1% outlier channels x8",
            "cache_instances": r32["instances"],
            "cache_bytes_total": r32["cache_bytes"],
            "timing": "K steps captured in one HIP graph; one untimed warm replay, then 5 timed replays of exactly "
            "K steps each between HIP timing events on the launch stream (created with hipEventDisableSystemFence: "
            "no cache writeback at the events), ms_per_step their median (a ~100 us spin kernel queued before "
            "each start event keeps host submission out of the timed region)",
        },
        "us_per_step": round(r32["us_per_step"], 3),
        **_step_detail(r32),
        "frac_of_peak": round(r32["gbs"] / HBM_PEAK_GBS, 4),
        "roofline": {
            "bound": "hbm",
            "achieved": round(r32["kernel_gbs"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(r32["kernel_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "kernel": "rec::decode_kernel<8, 8, 4, true> (fused append + split-K attention partials)",
            "kernel_us": round(r32["kernel_us"], 3),
            "algorithmic_bytes_per_launch": r32["bytes_per_launch"],
            "timing": "HIP timing events (no system-scope fence) around each of 5 replays (after a warm one) "
                      "of a graph of K launches of the kernel; the median",
        },
        "cpu_baseline": cpu,
    }
    if r1k is not None:
        result["context_1k_tiny"] = {
            "context": 1024,
            "q_heads": 8,
            "kv_heads": 1,
            "kv_format": "int8 symmetric, fp16 scale per (token, head); N(0, 1) K/V",
            "note": "the CPU-sized parity configuration; 64 instances (17 MB) fit the MALL, so the figure is "
                    "launch latency, not HBM streaming",
            "us_per_step": round(r1k["us_per_step"], 3),
            **_step_detail(r1k),
            "gbs": round(r1k["gbs"], 2),
            "kernel_us": round(r1k["kernel_us"], 3),
            "bytes_per_step": r1k["bytes_per_step"],
            "cache_instances": r1k["instances"],
        }
    if r252 is not None:
        result["context_252k"] = {
            "context": 258048,
            "us_per_step": round(r252["us_per_step"], 3),
            **_step_detail(r252),
            "gbs": round(r252["gbs"], 2),
            "frac_of_peak": round(r252["gbs"] / HBM_PEAK_GBS, 4),
            "kernel_us": round(r252["kernel_us"], 3),
            "kernel_gbs": round(r252["kernel_gbs"], 2),
            "kernel_frac_of_peak": round(r252["kernel_gbs"] / HBM_PEAK_GBS, 4),
            "bytes_per_step": r252["bytes_per_step"],
            "cache_instances": r252["instances"],
            "traffic": traffic_of("252k_int8"),
        }
    if rb4 is not None:
        result["context_32k_batch4"] = {
            "context": 32768,
            "batch": 4,
            "note": "informational: 4 sequences per step, the metric's configuration is batch 1",
            "us_per_step": round(rb4["us_per_step"], 3),
            **_step_detail(rb4),
            "gbs": round(rb4["gbs"], 2),
            "frac_of_peak": round(rb4["gbs"] / HBM_PEAK_GBS, 4),
            "kernel_us": round(rb4["kernel_us"], 3),
            "kernel_gbs": round(rb4["kernel_gbs"], 2),
            "kernel_frac_of_peak": round(rb4["kernel_gbs"] / HBM_PEAK_GBS, 4),
            "bytes_per_step": rb4["bytes_per_step"],
            "cache_instances": rb4["instances"],
        }
    if r4 is not None:
        result["context_131k_int4"] = {
            "context": 131072,
            "kv_format": "uint4 asymmetric, fp16 scale + zero-point per 32 dims; 5% Student-t(3) channels",
            "us_per_step": round(r4["us_per_step"], 3),
            **_step_detail(r4),
            "gbs": round(r4["gbs"], 2),
            "frac_of_peak": round(r4["gbs"] / HBM_PEAK_GBS, 4),
            "kernel_us": round(r4["kernel_us"], 3),
            "kernel_gbs": round(r4["kernel_gbs"], 2),
            "kernel_frac_of_peak": round(r4["kernel_gbs"] / HBM_PEAK_GBS, 4),
            "bytes_per_step": r4["bytes_per_step"],
            "cache_instances": r4["instances"],
            "traffic": traffic_of("131k_uint4"),
        }
    if raf is not None:
        result["context_32k_affine"] = {
            "context": 32768,
            "kv_format": "MLX-style affine group 64: 8-bit K, 4-bit V, bf16 scale + bias (the reference's default)",
            "us_per_step": round(raf["us_per_step"], 3),
            **_step_detail(raf),
            "gbs": round(raf["gbs"], 2),
            "frac_of_peak": round(raf["gbs"] / HBM_PEAK_GBS, 4),
            "kernel_us": round(raf["kernel_us"], 3),
            "kernel_gbs": round(raf["kernel_gbs"], 2),
            "kernel_frac_of_peak": round(raf["kernel_gbs"] / HBM_PEAK_GBS, 4),
            "bytes_per_step": raf["bytes_per_step"],
            "cache_instances": raf["instances"],
        }
    if raf252 is not None:
        result["context_252k_affine"] = {
            "context": 258048,
            "kv_format": "MLX-style affine group 64: 8-bit K, 4-bit V, bf16 scale + bias (the reference's default)",
            "us_per_step": round(raf252["us_per_step"], 3),
            **_step_detail(raf252),
            "gbs": round(raf252["gbs"], 2),
            "frac_of_peak": round(raf252["gbs"] / HBM_PEAK_GBS, 4),
            "kernel_us": round(raf252["kernel_us"], 3),
            "kernel_gbs": round(raf252["kernel_gbs"], 2),
            "kernel_frac_of_peak": round(raf252["kernel_gbs"] / HBM_PEAK_GBS, 4),
            "bytes_per_step": raf252["bytes_per_step"],
            "cache_instances": raf252["instances"],
        }
    for name, c in cpu_more.items():
        result[name]["cpu_baseline"] = c
    result.update(rbf)
    if rq4 is not None:
        result["q4_gemv"] = dict(
            format="MLX affine 4-bit, group 64, bf16 scales and biases; one bf16 vector, bf16 out",
            shapes=rq4,
            kernel="rec::q4_gemv_kernel (bf16 MFMA 16x16x32)",
        )
        result["q4_gemm_prefill"] = dict(
            format="the same packed matrix, 2,048 bf16 rows of x (a prefill chunk's projection), bf16 out",
            shapes=rq4m,
            kernel="rec::q4_xsum_kernel + rec::q4_gemm_kernel (bf16 MFMA 16x16x32)",
        )
    if rpf is not None:
        result["prefill_65536_plus_2048"] = rpf
    if rpf_short is not None:
        result["prefill_32768_plus_20"] = rpf_short
    if rpf_short_u4 is not None:
        result["prefill_32768_plus_20_uint4"] = rpf_short_u4
    if rpf_few is not None:
        result["prefill_65536_plus_4"] = rpf_few
    if rpf_few_affine is not None:
        result["prefill_65536_plus_4_affine"] = rpf_few_affine
    if rpf_few_u4 is not None:
        result["prefill_65536_plus_4_uint4"] = rpf_few_u4
    for fmt, r in rpf_fmt.items():
        result[f"prefill_65536_plus_2048_{fmt}"] = r
    if sliding is not None:
        result["sliding_window_513"] = sliding
    if floor is not None:
        result["read_floor"] = dict(
            floor,
            note="rec_stream_read: a plain streaming read of the configuration's K/V bytes in one launch, the "
                 "practical ceiling the decode kernel's roofline fraction is read against")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
