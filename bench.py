"""Benchmark of the packed-ternary hot path on one MI355X.

Headline (``value``): the decode GEMV (K2) at the north-star shape, Llama-3-8B
gate 4096 -> 14336, M = 1 token, bf16 activations, in HBM GB/s of algorithmic
bytes.  A "step" is one GEMV call on a fresh weight matrix: the weights rotate
through enough copies (> 2x the 256 MB Infinity Cache) that every call streams
from HBM, and the launches of a round are captured in a HIP graph so that the
GPU runs them back to back.  Inputs are resident in HBM before timing starts.

Also reported: the prefill GEMM (K3) at M = 2048 tokens, gate_up 4096 -> 28672
(TFLOP/s against the dense bf16 MFMA peak), K1 pack at 8192 x 3072, and the
reference CPU gemm_ternary (oracle/_ref, compiled from the reference sources)
timed on a bounded sample of the same GEMV workload on this host.

Prints ONE JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0       # dense bf16 MFMA
INT8_PEAK_TOPS = 5000.0         # dense int8 MFMA
MALL_BYTES = 256 << 20

METRIC = ("ternary GEMV HBM GB/s (% of peak) + prefill GEMM TFLOP/s (% MFMA peak), 1 GPU")


def log(msg: str) -> None:
    sys.stderr.write(f"[bench] {msg}\n")
    sys.stderr.flush()


def gemv_bytes(m: int, n: int, k: int, x_bytes: int = 2, beta: bool = False,
               bias: bool = False) -> int:
    """16*N*ceil(K/48) packed weights + activations + C write (+ C read) (+ bias)."""
    limbs = (k + 47) // 48
    return 16 * n * limbs + x_bytes * m * k + 4 * m * n * (2 if beta else 1) + (4 * n if bias else 0)


def make_weights(torch, ops, lib, n: int, k: int, copies: int, dev, seed: int):
    g = torch.Generator(dev).manual_seed(seed)
    out = []
    for _ in range(copies):
        w = torch.randn((n, k), generator=g, device=dev)   # effective W/0.02 ~ N(0, 1)
        out.append(ops.quantize_pack(w, 0.45, lib.THR_CPP))
        del w
    return out


def _capture(torch, launch, items, stream):
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for b in items:
            launch(b)
    return graph


def time_graph(torch, launch, buffers, steps: int, warmup: int, dist: bool = False,
               min_launches: int = 100, min_ms: float = 50.0, min_graph: int = 128):
    """Times exactly `steps` launches of `launch`, rotating through `buffers`, captured in
    HIP graphs so the GPU runs them back to back on one stream: a graph of at least
    `min_graph` launches cycling through the buffers (a whole number of rotations; a graph
    replay costs ~10-20 us at its boundary on this runtime, so a graph holds many launches),
    replayed steps // its size times, plus one graph of the remaining launches.
    `warmup` untimed launches (whole rotations) run first, then a synchronisation, then one
    more untimed rotation ahead of the start event (the graph of the remaining launches is
    replayed once untimed too, so no timed replay is a first one); the timed region ends with a
    synchronisation and is timed with HIP events on the launch stream.  Returns ms per
    launch; with dist=True a dict that adds the spread: each replay of the rotation graph
    timed on its own, over at least `min_launches` launches and `min_ms` of GPU time
    (median / p10 / p90 of the per-launch time)."""
    import numpy as np

    steps = max(1, int(steps))
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for i in range(min(max(warmup, 1), len(buffers))):   # eager warm-up, no capture
            launch(buffers[i])
    torch.cuda.synchronize()
    buffers = list(buffers) * max(1, -(-min_graph // len(buffers)))
    n = len(buffers)
    full = _capture(torch, launch, buffers, stream)
    rest = _capture(torch, launch, buffers[: steps % n], stream) if steps % n else None
    torch.cuda.synchronize()
    for _ in range(-(-warmup // n)):
        full.replay()
    if rest is not None:          # the partial graph's first replay is not timed either
        rest.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        # one untimed rotation ahead of the start event keeps the GPU busy while the host
        # submits the timed graphs, so the region holds the K launches back to back and
        # not the host's graph-launch latency
        full.replay()
        start.record(stream)
        for _ in range(steps // n):
            full.replay()
        if rest is not None:
            rest.replay()
        end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    if not dist:
        return ms
    reps = max(3, -(-min_launches // n), int(np.ceil(min_ms / max(ms * n, 1e-6))))
    events = []
    with torch.cuda.stream(stream):
        for _ in range(reps):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            full.replay()
            b.record(stream)
            events.append((a, b))
    torch.cuda.synchronize()
    per = np.array([a.elapsed_time(b) / n for a, b in events])
    return {"ms": ms, "timed_launches": steps, "mean_ms": float(per.mean()),
            "median_ms": float(np.median(per)), "p10_ms": float(np.percentile(per, 10)),
            "p90_ms": float(np.percentile(per, 90)), "samples": reps,
            "launches_per_sample": n}


def time_eager(torch, launch, n: int, steps: int, warmup: int, ahead: int = 64,
               min_launches: int = 100, min_ms: float = 50.0) -> dict:
    """Times exactly `steps` launches issued one by one on one stream (launch(i, stream)
    enqueues launch i on the stream handle, i indexing rotating buffers modulo n; meant for
    a direct C ABI call, which the host issues faster than the GPU runs it).  `warmup` untimed launches and a
    synchronisation come first, then the spread samples (repeats of the region below over
    32 launches); then `ahead` untimed launches keep the GPU busy while the host issues the
    timed ones, and HIP events on the stream bracket exactly the `steps` timed launches; a
    synchronisation ends the region.  Unlike a graph replay, the region
    holds no graph-launch boundary (~10-20 us on this runtime, which 20 launches would carry
    as ~0.5-1 us each).  Returns the same dict as time_graph(dist=True): the timed region's
    ms per launch, and the spread over repeats of the region (median / p10 / p90)."""
    import numpy as np

    steps = max(1, int(steps))
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    sh = stream.cuda_stream
    idx = 0
    for _ in range(max(warmup, 1)):
        launch(idx % n, sh)
        idx += 1
    torch.cuda.synchronize()

    def region(k):
        nonlocal idx
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        first = idx
        for i in range(first, first + ahead):
            launch(i % n, sh)
        a.record(stream)
        for i in range(first + ahead, first + ahead + k):
            launch(i % n, sh)
        b.record(stream)
        idx = first + ahead + k
        torch.cuda.synchronize()
        return a.elapsed_time(b) / k

    # the spread samples first: they also bring the clocks and caches to their loaded state
    # before the timed region, which runs last
    per = []
    total = 0.0
    while len(per) < 3 or len(per) * 32 < min_launches or total < min_ms:
        t = region(32)
        per.append(t)
        total += 32 * t
    per = np.array(per)
    ms = region(steps)
    return {"ms": ms, "timed_launches": steps, "mean_ms": float(per.mean()),
            "median_ms": float(np.median(per)), "p10_ms": float(np.percentile(per, 10)),
            "p90_ms": float(np.percentile(per, 90)), "samples": len(per),
            "launches_per_sample": 32}


def abi_launch(lib, x, x_dtype: int, wbufs, out, m: int, n: int, k: int, which: int = 3,
               alpha: float = 1.0, beta: float = 0.0, torch=None):
    """launch(i, stream) for time_eager: t81_hip_ternary_matmul_ws (which = 0, 2 or 3) on
    weight copy i, with a workspace of the size the shape asks for allocated once here (the
    C ABI call every consumer of the library makes; out is C, read when beta != 0)."""
    L = lib.lib()
    fn = L.t81_hip_ternary_matmul_ws
    wptrs = [w.data_ptr() for w in wbufs]
    xp, op = x.data_ptr(), out.data_ptr()
    need = int(L.t81_hip_ternary_matmul_workspace_size(m, n, k, x_dtype))
    ws = None
    if need > 0:
        ws = torch.empty(need, dtype=torch.uint8, device=out.device)
    wsp = ws.data_ptr() if ws is not None else None

    def launch(i, sh, ws=ws):
        rc = fn(which, xp, x_dtype, wptrs[i], op, m, n, k, alpha, beta, None, wsp, need, sh)
        if rc != 0:
            lib.check(rc)
    return launch


def spread_us(d: dict) -> dict:
    """The spread of a time_graph(dist=True) result, in microseconds."""
    return {"median_us": d["median_ms"] * 1e3, "p10_us": d["p10_ms"] * 1e3,
            "p90_us": d["p90_ms"] * 1e3, "mean_us": d["mean_ms"] * 1e3,
            "samples": d["samples"], "launches_per_sample": d["launches_per_sample"]}


def sha256_tensors(torch, *tensors) -> str:
    """SHA-256 over the bytes of the given (device or host) tensors, in order."""
    import hashlib

    h = hashlib.sha256()
    for t in tensors:
        h.update(t.detach().contiguous().view(-1).view(torch.uint8).cpu().numpy().tobytes())
    return h.hexdigest()


def cpu_threads() -> int:
    """Host threads for the all-core CPU baselines: the cores this process may use, at most
    16 (a GPU box's CPU share per GPU)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def _reference_lib():
    """(library, kind): the reference's own compiled CPU path (oracle/_ref), else the
    oracle's C restatement."""
    import oracle

    ref = oracle.ref()
    if ref is None:
        ref = oracle.ref("generic")
    return (ref, "reference") if ref is not None else (None, "port")


def cpu_limb_gemm(wp, xp, n_tok: int, k: int, budget_s: float, threads: int = 1) -> dict:
    """The reference CPU gemm_ternary (oracle/_ref: gemm_ternary_cpu_impl compiled from the
    reference's sources; the oracle's C restatement where that is not built) over weight
    rows wp (rows x L x 16) times the packed activation columns xp (L x n_tok x 16), in
    blocks of 16 rows spread over `threads` host threads (ctypes releases the GIL, so the
    blocks run in parallel), until every row is done or `budget_s` has passed.  Returns
    rows done, seconds and limb products per second."""
    import threading

    import numpy as np

    import oracle

    ref, kind = _reference_lib()
    rows = wp.shape[0]
    limbs = wp.shape[1]
    c = np.zeros((rows, n_tok), np.float32)
    block = 16
    nxt = [0]
    done = [0]
    lock = threading.Lock()
    t0 = time.perf_counter()

    def worker():
        while True:
            with lock:
                if nxt[0] >= rows or time.perf_counter() - t0 >= budget_s:
                    return
                r0 = nxt[0]
                nxt[0] = min(rows, r0 + block)
            r1 = min(rows, r0 + block)
            if kind == "reference":
                ref.gemm_ternary_rows(wp, xp, c, rows, n_tok, limbs * 48, r0, r1)
            else:
                c[r0:r1] = oracle.gemm_limb(wp[r0:r1], xp, c[r0:r1], r1 - r0, n_tok, limbs * 48)
            with lock:
                done[0] += r1 - r0

    pool = [threading.Thread(target=worker) for _ in range(threads)]
    for t in pool:
        t.start()
    for t in pool:
        t.join()
    dt = time.perf_counter() - t0
    products = done[0] * limbs * n_tok
    return {"kind": kind, "rows": done[0], "seconds": dt, "limb_products": products,
            "limb_products_per_s": products / dt, "threads": threads,
            "variant": ref.variant if kind == "reference" else "oracle C restatement",
            "simd": ref.simd_path() if kind == "reference" else "scalar"}


def _gemv_inputs(n: int, k: int, n_tok: int, seed: int):
    import numpy as np

    import oracle

    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k)).astype(np.float32)
    wp = oracle.pack_rows(w, 0.45, 0)                                       # (n, L, 16)
    x = rng.standard_normal((n_tok, k)).astype(np.float32)
    xp = oracle.pack_cols(x, np.float32(oracle.torch_threshold(0.5)), 1)    # (L, n_tok, 16)
    return wp, xp


def cpu_reference_gemv(n: int, k: int, budget_s: float, threads: int = 1):
    """The GEMV workload (W n x L limbs times one packed activation column) on the
    reference CPU path.  Returns (GB/s of packed weights streamed, detail)."""
    wp, xp = _gemv_inputs(n, k, 1, seed=0)
    d = cpu_limb_gemm(wp, xp, 1, k, budget_s, threads)
    limbs = wp.shape[1]
    return 16 * d["rows"] * limbs / d["seconds"] / 1e9, d


def cpu_reference_gemm(m: int, n: int, k: int, rows: int, tokens: int, budget_s: float,
                       threads: int = 1):
    """The prefill GEMM workload sampled: `rows` weight rows x `tokens` activation columns
    of the m x n x k problem on the reference CPU path, extrapolated linearly in
    m * n * L limb products.  Returns (TFLOP/s-equivalent of the full GEMM, detail)."""
    wp, xp = _gemv_inputs(rows, k, tokens, seed=1)
    d = cpu_limb_gemm(wp, xp, tokens, k, budget_s, threads)
    limbs = wp.shape[1]
    full_s = m * n * limbs / d["limb_products_per_s"]
    d["extrapolated_full_s"] = full_s
    return 2.0 * m * n * k / full_s / 1e12, d


def cpu_pack(rows: int, cols: int, threads: int = 1, reps: int = 3):
    """K1's workload on the CPU: the oracle's single-thread restatement of
    pack_dense_matrix (python/bindings.cpp:497-515) over a rows x cols float32 matrix,
    split into row blocks over `threads` threads; median of `reps` runs.  Returns
    (GB/s of algorithmic bytes, seconds)."""
    import threading

    import numpy as np

    import oracle

    w = (np.random.default_rng(2).standard_normal((rows, cols)) * 0.02).astype(np.float32)
    bounds = np.linspace(0, rows, threads + 1).astype(int)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        pool = [threading.Thread(target=oracle.pack_rows, args=(w[a:b], 0.45, 0))
                for a, b in zip(bounds[:-1], bounds[1:])]
        for t in pool:
            t.start()
        for t in pool:
            t.join()
        times.append(time.perf_counter() - t0)
    sec = float(np.median(times))
    nbytes = 4 * rows * cols + 16 * rows * ((cols + 47) // 48)
    return nbytes / sec / 1e9, sec


# ------------------------------------------------------- config 5: decoder stack --
# A Llama-3-8B-shaped decoder whose four projections per layer are t8.nn.Linear
# (t81lib_amd.nn.Linear, eval mode: packed once, then K2 / K3 per call); RMSNorm,
# RoPE, attention and the lm_head stay dense torch code, as the config leaves them.
# Attention runs in float32 on a float32 KV cache (keys stored transposed), so every
# batched product has contiguous or sliced -- never transposed -- operands.

LLAMA3_8B = dict(layers=32, hidden=4096, heads=32, kv_heads=8, ffn=14336, vocab=128256)


class DecoderStack:
    """Random-init ternary decoder: weights ~ N(0, 1) (the effective W / 0.02, so the
    0.45 threshold leaves ~1/3 zero trits; literal N(0, 0.02) weights would all be zero),
    embedding and lm_head ~ N(0, 0.02) in bf16.  ``reference=True`` replaces each packed
    linear by F.linear in float32 with the same trits (the test oracle of the stack);
    ``reference="split"`` does the same with K summed as two halves, a second float32
    summation order (the tests use its distance from the first as the scale of rounding
    drift through the stack)."""

    def __init__(self, torch, dev, layers, hidden, heads, kv_heads, ffn, vocab, max_batch,
                 max_tokens, seed=0, reference=False):
        from t81lib_amd import nn as t8nn
        from t81lib_amd import ops

        self.t = torch
        self.F = torch.nn.functional
        self.hidden, self.heads, self.kv_heads, self.ffn = hidden, heads, kv_heads, ffn
        self.hd = hidden // heads
        self.group = heads // kv_heads
        self.reference = reference
        g = torch.Generator(dev).manual_seed(seed)
        shapes = {"qkv": (hidden, hidden + 2 * kv_heads * self.hd), "o": (hidden, hidden),
                  "gate_up": (hidden, 2 * ffn), "down": (ffn, hidden)}
        self.blocks = []
        for _ in range(layers):
            blk = {}
            for name, (fin, fout) in shapes.items():
                lin = t8nn.Linear(fin, fout, bias=False, device=dev)
                with torch.no_grad():
                    lin.weight.copy_(torch.randn((fout, fin), generator=g, device=dev))
                lin.eval()
                with torch.no_grad():   # pack now (K1), outside any timed region
                    lin(torch.zeros((1, fin), dtype=torch.bfloat16, device=dev))
                if reference:
                    tw = lin.ternary_weight
                    blk[name] = ops.unpack(tw.packed, fout, fin).float()
                else:
                    blk[name] = lin
            blk["n1"] = torch.ones(hidden, dtype=torch.bfloat16, device=dev)
            blk["n2"] = torch.ones(hidden, dtype=torch.bfloat16, device=dev)
            self.blocks.append(blk)
        self.norm = torch.ones(hidden, dtype=torch.bfloat16, device=dev)
        self.embed = (torch.randn((vocab, hidden), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        self.lm_head_t = (torch.randn((hidden, vocab), generator=g, device=dev) * 0.02).to(
            torch.bfloat16)
        # float32 KV cache: keys as (B, kv_heads, hd, T), values as (B, kv_heads, T, hd)
        self.kt = [torch.zeros((max_batch, kv_heads, self.hd, max_tokens), device=dev)
                   for _ in range(layers)]
        self.v = [torch.zeros((max_batch, kv_heads, max_tokens, self.hd), device=dev)
                  for _ in range(layers)]
        inv = 1.0 / (500000.0 ** (torch.arange(0, self.hd, 2, device=dev).float() / self.hd))
        ang = torch.arange(max_tokens, device=dev).float()[:, None] * inv[None, :]
        self.cos, self.sin = ang.cos(), ang.sin()            # (T, hd / 2)

    def _linear(self, blk, name, x2d):
        if self.reference == "split":
            h = x2d.shape[-1] // 2
            xf, wt = x2d.float(), blk[name]
            return self.F.linear(xf[:, :h], wt[:, :h]) + self.F.linear(xf[:, h:], wt[:, h:])
        if self.reference:
            return self.F.linear(x2d.float(), blk[name])
        return blk[name](x2d)

    def _rmsnorm(self, x, w):
        xf = x.float()
        return (xf * self.t.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(x.dtype) * w

    def _rope(self, x, pos0):           # x (B, S, nh, hd) float32
        s = x.shape[1]
        c = self.cos[pos0:pos0 + s][None, :, None, :]
        sn = self.sin[pos0:pos0 + s][None, :, None, :]
        x1, x2 = x[..., : self.hd // 2], x[..., self.hd // 2:]
        return self.t.cat([x1 * c - x2 * sn, x2 * c + x1 * sn], dim=-1)

    def forward(self, tokens, pos0: int):
        """tokens (B, S) -> float32 logits of the last position (B, vocab)."""
        t = self.t
        B, S = tokens.shape
        H, KV, hd, G = self.hidden, self.kv_heads, self.hd, self.group
        x = self.embed[tokens]                                    # (B, S, H) bf16
        T = pos0 + S
        for li, blk in enumerate(self.blocks):
            h = self._rmsnorm(x, blk["n1"]).reshape(B * S, H)
            qkv = self._linear(blk, "qkv", h)                     # float32
            q = self._rope(qkv[:, :H].reshape(B, S, self.heads, hd), pos0)
            k = self._rope(qkv[:, H:H + KV * hd].reshape(B, S, KV, hd), pos0)
            v = qkv[:, H + KV * hd:].reshape(B, S, KV, hd)
            self.kt[li][:B, :, :, pos0:T] = k.permute(0, 2, 3, 1)
            self.v[li][:B, :, pos0:T, :] = v.permute(0, 2, 1, 3)
            qg = q.reshape(B, S, KV, G, hd).permute(0, 2, 3, 1, 4).reshape(B, KV, G * S, hd)
            scores = t.matmul(qg, self.kt[li][:B, :, :, :T]) * (1.0 / hd ** 0.5)
            if S > 1:
                qpos = pos0 + t.arange(G * S, device=x.device) % S
                mask = t.arange(T, device=x.device)[None, :] > qpos[:, None]
                scores = scores.masked_fill(mask, float("-inf"))
            att = t.matmul(t.softmax(scores, dim=-1), self.v[li][:B, :, :T, :])
            att = att.reshape(B, KV, G, S, hd).permute(0, 3, 1, 2, 4).reshape(B * S, H)
            x = x + self._linear(blk, "o", att.to(t.bfloat16)).reshape(B, S, H).to(t.bfloat16)
            h2 = self._rmsnorm(x, blk["n2"]).reshape(B * S, H)
            gu = self._linear(blk, "gate_up", h2)
            act = (self.F.silu(gu[:, : self.ffn]) * gu[:, self.ffn:]).to(t.bfloat16)
            x = x + self._linear(blk, "down", act).reshape(B, S, H).to(t.bfloat16)
        xl = self._rmsnorm(x[:, -1], self.norm)                   # (B, H) bf16
        return t.matmul(xl, self.lm_head_t).float()

    def decode_static(self, tok, pos):
        """One decode step with shapes that do not depend on the position, so it can be
        captured in a graph: tok (B, 1) token ids, pos a one-element device tensor.  The
        step attends over the whole cache with the slots past pos masked out."""
        t = self.t
        B = tok.shape[0]
        H, KV, hd, G = self.hidden, self.kv_heads, self.hd, self.group
        tmax = self.kt[0].shape[3]
        x = self.embed[tok]                                       # (B, 1, H)
        c = self.cos.index_select(0, pos)[None, :, None, :]
        sn = self.sin.index_select(0, pos)[None, :, None, :]

        def rope(v):
            v1, v2 = v[..., : hd // 2], v[..., hd // 2:]
            return t.cat([v1 * c - v2 * sn, v2 * c + v1 * sn], dim=-1)

        mask = t.arange(tmax, device=tok.device)[None, :] > pos[:, None]      # (1, tmax)
        for li, blk in enumerate(self.blocks):
            h = self._rmsnorm(x, blk["n1"]).reshape(B, H)
            qkv = self._linear(blk, "qkv", h)
            q = rope(qkv[:, :H].reshape(B, 1, self.heads, hd))
            k = rope(qkv[:, H:H + KV * hd].reshape(B, 1, KV, hd))
            v = qkv[:, H + KV * hd:].reshape(B, 1, KV, hd)
            kt, vc = self.kt[li][:B], self.v[li][:B]
            kt.index_copy_(3, pos, k.permute(0, 2, 3, 1).contiguous())
            vc.index_copy_(2, pos, v.permute(0, 2, 1, 3).contiguous())
            qg = q.reshape(B, KV, G, hd)
            scores = (t.matmul(qg, kt) * (1.0 / hd ** 0.5)).masked_fill(mask, float("-inf"))
            att = t.matmul(t.softmax(scores, dim=-1), vc).reshape(B, H)
            x = x + self._linear(blk, "o", att.to(t.bfloat16)).reshape(B, 1, H).to(t.bfloat16)
            h2 = self._rmsnorm(x, blk["n2"]).reshape(B, H)
            gu = self._linear(blk, "gate_up", h2)
            act = (self.F.silu(gu[:, : self.ffn]) * gu[:, self.ffn:]).to(t.bfloat16)
            x = x + self._linear(blk, "down", act).reshape(B, 1, H).to(t.bfloat16)
        xl = self._rmsnorm(x[:, -1], self.norm)
        return t.matmul(xl, self.lm_head_t).float()

    def decode_graph(self, batch):
        """A captured greedy decode step for `batch` sequences: returns (graph, token
        buffer, position tensor, logits).  Set the token buffer to the last tokens and the
        position to theirs; each replay writes the step's logits, puts the argmax in the
        token buffer and advances the position."""
        t = self.t
        dev = self.embed.device
        tok = t.zeros((batch, 1), dtype=t.long, device=dev)
        pos = t.zeros((1,), dtype=t.long, device=dev)
        side = t.cuda.Stream()
        side.wait_stream(t.cuda.current_stream())
        with t.cuda.stream(side):
            self.decode_static(tok, pos)                          # warm-up outside capture
        t.cuda.current_stream().wait_stream(side)
        t.cuda.synchronize()
        graph = t.cuda.CUDAGraph()
        with t.cuda.graph(graph):
            logits = self.decode_static(tok, pos)
            tok.copy_(logits.argmax(-1, keepdim=True))
            pos.add_(1)
        return graph, tok, pos, logits


def run_stack(torch, dev, prompt=1024, steps=256, batches=(1, 32)) -> dict:
    """Config 5: prompt of 1024 random token ids per sequence, then 256 greedy decode
    steps, at batch 1 and 32; tokens/s of prefill (eager) and of decode (each step one
    replay of a captured graph)."""
    cfg = LLAMA3_8B
    t0 = time.perf_counter()
    st = DecoderStack(torch, dev, cfg["layers"], cfg["hidden"], cfg["heads"], cfg["kv_heads"],
                      cfg["ffn"], cfg["vocab"], max(batches), prompt + steps, seed=9)
    torch.cuda.synchronize()
    log(f"stack built ({cfg['layers']} layers, weights packed) in {time.perf_counter() - t0:.1f} s")
    out = {"workload": "config 5: Llama-3-8B-shaped 32-layer decoder, t8.nn.Linear projections "
                       "(K1 pack, K2 / K3 matmul), dense bf16 embedding / lm_head / RMSNorm, "
                       "float32 attention and KV cache, random token ids, greedy; prefill eager, "
                       "decode steps replayed from a captured graph",
           "prompt": prompt, "decode_steps": steps, "results": []}
    g = torch.Generator(dev).manual_seed(10)
    with torch.no_grad():
        st.forward(torch.randint(0, cfg["vocab"], (1, 16), generator=g, device=dev), 0)  # warm-up
        for b in batches:
            graph, tok, pos, _ = st.decode_graph(b)   # before the prompt fills the cache
            tokens = torch.randint(0, cfg["vocab"], (b, prompt), generator=g, device=dev)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            logits = st.forward(tokens, 0)
            torch.cuda.synchronize()
            t_pre = time.perf_counter() - t1
            tok.copy_(logits.argmax(-1, keepdim=True))
            pos.fill_(prompt)
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            for _ in range(steps):
                graph.replay()
            torch.cuda.synchronize()
            t_dec = time.perf_counter() - t2
            r = {"batch": b, "prefill_s": t_pre, "prefill_tokens_per_s": b * prompt / t_pre,
                 "decode_s": t_dec, "decode_tokens_per_s": b * steps / t_dec,
                 "decode_ms_per_step": t_dec / steps * 1e3}
            out["results"].append(r)
            log(f"stack batch {b}: prefill {b * prompt} tokens in {t_pre * 1e3:.1f} ms "
                f"({r['prefill_tokens_per_s']:.0f} tok/s), decode {steps} steps in "
                f"{t_dec:.2f} s ({r['decode_tokens_per_s']:.0f} tok/s, "
                f"{r['decode_ms_per_step']:.2f} ms/step)")
            del graph
    del st
    torch.cuda.empty_cache()
    return out


def run_spmm(torch, dev) -> list:
    """spmm_simple on the reference example's shape (256 x 256, 3 %, N = 128) and on the
    Llama gate shape at the same density: plan = stable row sort (timed once), apply = the
    hot kernel (graph-timed).  Unique bytes: 12 per entry + row_ptr + B + C."""
    from t81lib_amd import sparse
    out = []
    for name, srows, scols, n_feat in (("example 256x256", 256, 256, 128),
                                       ("llama.gate 14336x4096", 14336, 4096, 128)):
        nnz = int(srows * scols * 0.03)
        g = torch.Generator(dev).manual_seed(8)
        vals = torch.randint(-3, 4, (nnz,), generator=g, device=dev)
        ri = torch.randint(0, srows, (nnz,), generator=g, device=dev, dtype=torch.int32)
        ci = torch.randint(0, scols, (nnz,), generator=g, device=dev, dtype=torch.int32)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        A = sparse.SparseTernaryMatrix(vals, ri, ci, srows, scols)
        plan_ms = (time.perf_counter() - t0) * 1e3
        Bm = torch.randn((scols, n_feat), device=dev)
        outs = [torch.empty((srows, n_feat), device=dev) for _ in range(2)]
        ms = time_graph(torch, lambda c: A.matmul(Bm, c), outs, 256, 16)
        nbytes = 12 * nnz + 4 * (srows + 1) + 4 * scols * n_feat + 4 * srows * n_feat
        gbs = nbytes / (ms * 1e-3) / 1e9
        gather = 4.0 * nnz * n_feat / (ms * 1e-3) / 1e9
        out.append({"shape": f"spmm_simple {name} 3% N={n_feat}", "nnz": nnz, "us": ms * 1e3,
                    "GBps": gbs, "frac_hbm": gbs / HBM_PEAK_GBPS, "B_gather_GBps": gather,
                    "plan_ms": plan_ms})
        log(f"spmm {name} nnz={nnz} N={n_feat}: {ms * 1e3:7.2f} us  {gbs:6.0f} GB/s unique, "
            f"{gather:6.0f} GB/s B gathers; plan {plan_ms:6.2f} ms")
        A.close()
        del A, Bm, outs, vals, ri, ci
    torch.cuda.empty_cache()
    return out


def run_aux(torch, ops, _lib, dev) -> list:
    """The HBM-bound kernels off the GEMM path: the backend contract's elementwise ops
    (where / clamp / lerp / addcmul over 32 Mi float32 elements, 16 / 8 / 16 / 16 bytes per
    element) and the reference's TQ1_0 row codec on 8192 x 3072 float32 (quantize: 4 bytes
    per value in, 2 per 8 values out; dequantize: the reverse).  Two buffer sets, each
    larger than the MALL, alternate, so every launch streams from HBM; graph-timed, GB/s of
    algorithmic bytes and the fraction of 8 TB/s."""
    from t81lib_amd import gguf
    out = []
    n = 32 << 20
    sets = []
    for i in range(2):
        g = torch.Generator(dev).manual_seed(20 + i)
        sets.append([torch.randn(n, device=dev, generator=g) for _ in range(4)])

    def one(name, fn, nbytes, bufs):
        ms = time_graph(torch, fn, bufs, 200, 8)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out.append({"kernel": name, "us": ms * 1e3, "bytes": nbytes, "GBps": gbs,
                    "frac_hbm": gbs / HBM_PEAK_GBPS})
        log(f"aux {name}: {ms * 1e3:8.2f} us  {gbs:7.1f} GB/s  {gbs / HBM_PEAK_GBPS:.3f} of peak")

    one("where 32Mi float32", lambda b: ops.where(b[0], b[1], b[2], out=b[3]), 16 * n, sets)
    one("clamp 32Mi float32", lambda b: ops.clamp(b[0], -0.5, 0.5, out=b[3]), 8 * n, sets)
    one("lerp 32Mi float32", lambda b: ops.lerp(b[0], b[1], b[2], out=b[3]), 16 * n, sets)
    one("addcmul 32Mi float32", lambda b: ops.addcmul(b[0], b[1], b[2], 0.75, out=b[3]),
        16 * n, sets)
    del sets
    rows, cols = 8192, 3072
    L = _lib.lib()
    # per copy: source, scales, words, dequantized output (preallocated: the graphs hold the
    # kernels alone)
    bufs = []
    for _ in range(4):
        src = torch.randn((rows, cols), device=dev)
        sc, wd = gguf.quantize_rows_tq1_0(src)
        bufs.append((src, sc, wd, torch.empty((rows, cols), device=dev)))
    qb = 4 * rows * cols + 2 * rows * (cols // 8) + 4 * rows

    def quant(b):
        _lib.check(L.t81_hip_tq1_quantize_rows(b[0].data_ptr(), rows, cols, 0.45, None,
                                               b[1].data_ptr(), b[2].data_ptr(),
                                               torch.cuda.current_stream().cuda_stream))

    def dequant(b):
        _lib.check(L.t81_hip_tq1_dequantize_rows(b[2].data_ptr(), rows, cols, b[1].data_ptr(),
                                                 b[3].data_ptr(),
                                                 torch.cuda.current_stream().cuda_stream))
    one("TQ1_0 quantize rows 8192x3072 float32", quant, qb, bufs)
    one("TQ1_0 dequantize rows 8192x3072 float32", dequant, qb, bufs)
    # the tensor payload behind t81lib.dequant_tq1_0 (groups of 32 rows, half scales), and
    # the GGUF TQ1_0 / TQ2_0 blocks of 256 weights
    pb = int(L.t81_hip_tq1_payload_bytes(rows, cols, 32, 0))
    pays = [(torch.empty(pb, dtype=torch.uint8, device=dev), b[3], b[0]) for b in bufs]

    def quant_payload(b):
        _lib.check(L.t81_hip_tq1_quantize_payload(b[2].data_ptr(), rows, cols, 32, 0, 0.45,
                                                  b[0].data_ptr(),
                                                  torch.cuda.current_stream().cuda_stream))
    for b in pays:
        quant_payload(b)
    # the writer has no reference counterpart (the reference only reads payloads)
    one("TQ1_0 quantize payload 8192x3072 float32 (writer)", quant_payload,
        4 * rows * cols + pb, pays)

    def dequant_payload(b):
        _lib.check(L.t81_hip_tq1_dequantize_payload(b[0].data_ptr(), pb, rows, cols, 32, 0,
                                                    b[1].data_ptr(),
                                                    torch.cuda.current_stream().cuda_stream))
    one("TQ1_0 dequantize payload 8192x3072 float32", dequant_payload, 4 * rows * cols + pb,
        pays)
    for quant, name in ((34, "TQ1_0"), (35, "TQ2_0")):
        gb = rows * (cols // 256) * int(L.t81_hip_tq_block_bytes(quant))
        blks = []
        for b in bufs:
            blk = torch.empty(gb, dtype=torch.uint8, device=dev)
            _lib.check(L.t81_hip_tq_quantize(b[0].data_ptr(), blk.data_ptr(), rows, cols, 0.45,
                                             quant, torch.cuda.current_stream().cuda_stream))
            blks.append((blk, b[3], b[0]))

        def quant_blocks(b, quant=quant):
            _lib.check(L.t81_hip_tq_quantize(b[2].data_ptr(), b[0].data_ptr(), rows, cols, 0.45,
                                             quant, torch.cuda.current_stream().cuda_stream))

        def dequant_blocks(b, quant=quant):
            _lib.check(L.t81_hip_tq_dequantize(b[0].data_ptr(), b[1].data_ptr(), rows, cols,
                                               quant, torch.cuda.current_stream().cuda_stream))
        one(f"GGUF {name} quantize 8192x3072 float32", quant_blocks, 4 * rows * cols + gb,
            blks)
        one(f"GGUF {name} dequantize 8192x3072 float32", dequant_blocks,
            4 * rows * cols + gb, blks)
        del blks
    del bufs, pays
    torch.cuda.empty_cache()
    return out


DECODE_SHAPES = [("phi3.qkv", 3072, 9216), ("phi3.o", 3072, 3072), ("phi3.gate_up", 3072, 16384),
                 ("phi3.down", 8192, 3072), ("llama.gate", 4096, 14336),
                 ("llama.down", 14336, 4096)]


def run_decode(torch, ops, lib, dev, only_case=None) -> dict:
    """Config 3 (Phi-3 decode shapes) and the Llama-3-8B gate / down shapes at 1, 4, 8 and
    16 tokens, and at 32 (config 5's decode batch), 48 and 64, through the product path
    (ops.ternary_matmul: K2 up to 16 tokens, with the workspace its K splits use; the K3
    entry from 17, whose bf16 calls run K2's column-block stream kernel with two and three
    16-token blocks, two launches at 49..64, or the eight-wave kernel at 49..64 over K >
    8192): median microseconds per call over rotating weight copies (> 2 x MALL, so every
    call streams from HBM), GB/s of algorithmic bytes, and each shape's 16-token time over
    its one-token time.  The Llama shapes also with float32 activations at 1, 8 and 16..64
    tokens (keys f32_M*), the form t8.nn.Linear's float inputs take."""
    shapes = {}
    todo = DECODE_SHAPES if only_case is None else [("case", only_case[0], only_case[1])]
    for name, k, n in todo:
        wbytes = 16 * n * ((k + 47) // 48)
        copies = max(4, -(-2 * MALL_BYTES // wbytes) + 2)
        wb = make_weights(torch, ops, lib, n, k, copies, dev, seed=3)
        row = {"K": k, "N": n}
        runs = [("", torch.bfloat16, m) for m in
                ((1, 4, 8, 16, 32, 48, 64) if only_case is None else (only_case[2],))]
        if only_case is None and name.startswith("llama"):
            runs += [("f32_", torch.float32, m) for m in (1, 8, 16, 32, 48, 64)]
        for tag, dt, m in runs:
            x = torch.randn((m, k), device=dev).to(dt)
            out = torch.empty((m, n), device=dev)
            d = time_graph(torch, lambda w: ops.ternary_matmul(x, w, k, c=out), wb, 256, 32,
                           dist=True, min_launches=100, min_ms=20.0)
            us = d["median_ms"] * 1e3
            row[f"{tag}M{m}_us"] = round(us, 3)
            row[f"{tag}M{m}_GBps"] = round(gemv_bytes(m, n, k, 4 if tag else 2) / (us * 1e-6)
                                           / 1e9, 1)
            log(f"decode {name:13s} {tag or 'bf16_'}M={m:2d} {k:5d}->{n:5d}: {us:7.2f} us")
            del x, out
        if only_case is None:
            row["M16_over_M1"] = round(row["M16_us"] / row["M1_us"], 3)
        shapes[name] = row
        del wb
        torch.cuda.empty_cache()
    return {"workload": "K2 decode at 1-16 tokens (32, 48, 64: the K3 entry -- K2's "
                        "column-block kernel, or the eight-wave kernel at 64 over K > 8192), "
                        "bf16 x, fp32 out, alpha=1 beta=0, median over rotating weight copies; "
                        "config 3 (Phi-3) plus the Llama-3-8B gate / down shapes, those also "
                        "with float32 x at 1, 8 and 16-64 tokens (f32_M*)",
            "shapes": shapes}


def run_gemv_valu(torch, ops, lib, dev) -> dict:
    """The north-star form of K2 beside the matrix-core one, same box, same run: the one-token
    GEMV at 4096 -> 14336 (the headline shape) over the same rotating weight copies, as
    ops.ternary_matmul (K2: LDS-table decode, v_mfma_f32_16x16x32_bf16, LDS row sums) and as
    t81_floor_gemv_valu (the same table decode, v_dot2c_f32_bf16 products in each lane, DPP
    row sums per weight row, no matrix cores; csrc/floors.hip), best of 256-4096
    workgroups x 1, 2, 4 rows in flight per wave.  Integer activations (exact in bf16) make
    both outputs exact, so they must agree bit for bit; medians over graph replays."""
    import ctypes

    K, N = 4096, 14336
    wbytes = 16 * N * ((K + 47) // 48)
    copies = max(8, -(-2 * MALL_BYTES // wbytes) + 4)
    wbufs = make_weights(torch, ops, lib, N, K, copies, dev, seed=1)
    g = torch.Generator(dev).manual_seed(9)
    x = torch.randint(-64, 65, (1, K), generator=g, device=dev).to(torch.bfloat16)
    flib = ctypes.CDLL(os.path.join(ROOT, "t81lib_amd", "libt81_floors.so"))
    flib.t81_floor_gemv_valu.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_void_p]
    y_m = torch.empty((1, N), device=dev)
    y_v = torch.empty((1, N), device=dev)
    ops.ternary_matmul(x, wbufs[0], K, c=y_m, kernel=2)

    def valu(wb, blocks, depth):
        rc = flib.t81_floor_gemv_valu(x.data_ptr(), wb.data_ptr(), y_v.data_ptr(), N, K, blocks,
                                      depth, torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(f"t81_floor_gemv_valu failed ({rc})")

    valu(wbufs[0], 1024, 2)
    torch.cuda.synchronize()
    exact = bool(torch.equal(y_m.view(torch.int32), y_v.view(torch.int32)))
    mfma = time_graph(torch, lambda wb: ops.ternary_matmul(x, wb, K, c=y_m, kernel=2), wbufs,
                      256, 32, dist=True)
    best = None
    for blocks in (256, 512, 1024, 2048, 4096):
        for depth in (1, 2, 4):
            r = time_graph(torch, lambda wb: valu(wb, blocks, depth), wbufs, 256, 32, dist=True)
            if best is None or r["median_ms"] < best[2]["median_ms"]:
                best = (blocks, depth, r)
    blocks, depth, r = best
    out = {"workload": f"one-token GEMV {K}->{N}, bf16 integer-valued x, {copies} rotating "
                       f"weight copies",
           "mfma_us": mfma["median_ms"] * 1e3, "valu_us": r["median_ms"] * 1e3,
           "valu_config": {"workgroups": blocks, "rows_in_flight_per_wave": depth},
           "mfma_GBps": gemv_bytes(1, N, K) / (mfma["median_ms"] * 1e-3) / 1e9,
           "valu_GBps": gemv_bytes(1, N, K) / (r["median_ms"] * 1e-3) / 1e9,
           "valu_over_mfma": r["median_ms"] / mfma["median_ms"], "outputs_bit_identical": exact}
    log(f"gemv A/B {K}->{N}: matrix cores {out['mfma_us']:.2f} us, VALU {out['valu_us']:.2f} us "
        f"({blocks} workgroups, {depth} rows in flight), identical={exact}")
    del wbufs
    torch.cuda.empty_cache()
    return out


PREFILL_SHAPES = [("llama.qkv", 4096, 6144), ("llama.gate_up", 4096, 28672),
                  ("llama.down", 14336, 4096)]


def run_prefill(torch, ops, lib, dev) -> dict:
    """Config 4: the three Llama-3-8B prefill shapes at M = 512, 2048 and 8192 tokens, bf16
    activations ~ N(0,1), with (alpha, beta) = (1, 0) and (0.5, 1) over a float32 C ~ N(0,1)
    (read and written in place), through the C ABI (t81_hip_ternary_matmul_ws with the
    workspace the shape asks for): exactly 100 timed launches issued one by one after 20
    untimed ones, over two weight copies, plus >= 50 ms of spread samples.  TFLOP/s of 2 M N K and the fraction of the bf16
    matrix-core peak, from the mean over the 100 timed launches (median alongside)."""
    cases, f32_cases = [], []
    for name, k, n in PREFILL_SHAPES:
        wb = make_weights(torch, ops, lib, n, k, 2, dev, seed=4)
        for m in (512, 2048, 8192):
            x = torch.randn((m, k), device=dev).to(torch.bfloat16)
            c = torch.randn((m, n), device=dev)
            for alpha, beta in ((1.0, 0.0), (0.5, 1.0)):
                d = time_eager(torch, abi_launch(lib, x, lib.DTYPE_BF16, wb, c, m, n, k, which=3,
                                                 alpha=alpha, beta=beta, torch=torch),
                               len(wb), 100, 20, ahead=4)
                flops = 2.0 * m * n * k
                tf = flops / (d["ms"] * 1e-3) / 1e12
                cases.append({"shape": name, "M": m, "K": k, "N": n, "alpha": alpha, "beta": beta,
                              "ms": round(d["ms"], 5), "median_ms": round(d["median_ms"], 5),
                              "timed_launches": d["timed_launches"], "tflops": round(tf, 1),
                              "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                              "tokens_per_s_equiv": round(m / (d["ms"] * 1e-3))})
                log(f"prefill {name:14s} M={m:5d} a={alpha} b={beta}: {d['ms'] * 1e3:8.1f} us "
                    f"(median {d['median_ms'] * 1e3:8.1f})  {tf:7.1f} TFLOP/s  "
                    f"{tf / BF16_PEAK_TFLOPS:.3f}")
            del x, c
        # float32 activations at M = 2048, alpha 1 beta 0 (t8.nn.Linear's float inputs):
        # the planes through the workspace where they pay, else the eight-wave kernel
        m = 2048
        x = torch.randn((m, k), device=dev)
        c = torch.randn((m, n), device=dev)
        d = time_eager(torch, abi_launch(lib, x, lib.DTYPE_F32, wb, c, m, n, k, which=3,
                                         torch=torch), len(wb), 100, 20, ahead=4)
        tf = 2.0 * m * n * k / (d["ms"] * 1e-3) / 1e12
        f32_cases.append({"shape": name, "M": m, "K": k, "N": n, "ms": round(d["ms"], 5),
                          "median_ms": round(d["median_ms"], 5), "tflops": round(tf, 1),
                          "frac_of_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4)})
        log(f"prefill {name:14s} M={m:5d} float32 x: {d['ms'] * 1e3:8.1f} us  {tf:7.1f} TFLOP/s")
        del x, c
        del wb
        torch.cuda.empty_cache()
    return {"workload": "config 4: K3 prefill GEMM on the Llama-3-8B qkv / gate_up / down shapes "
                        "at M = 512, 2048, 8192, bf16 x, fp32 C, (alpha, beta) = (1, 0) and "
                        "(0.5, 1); 100 timed launches each; float32_x: the same shapes at "
                        "M = 2048 with float32 activations, alpha 1 beta 0",
            "peak_tflops": BF16_PEAK_TFLOPS, "cases": cases, "float32_x": f32_cases}


def run_limb(torch, ops, lib, dev, cpu_budget: float, with_cpu: bool) -> dict:
    """Config 1, the reference's own CPU case: gemm_ternary_cpu_impl's shape with the limb GEMM
    K4 (A = W as 1024 x 22 limbs, B = the column-packed activations 22 x 64, C 1024 x 64,
    alpha 1, beta 0): limb products per second over 100 timed launches, and the compiled
    reference timed on the same product in the same run."""
    M, N, K = 1024, 64, 1024
    kl = (K + 47) // 48
    A = make_weights(torch, ops, lib, M, K, 2, dev, seed=7)
    x = torch.randn((N, K), device=dev)
    B = ops.pack_cols(x, 0.5, lib.THR_TORCH)
    C = torch.zeros((M, N), device=dev)
    d = time_graph(torch, lambda a: ops.gemm_limb(a, B, C, M, N, kl * 48), A, 100, 10, dist=True)
    products = M * N * kl
    out = {"workload": "config 1: K4 limb GEMM in gemm_ternary_cpu_impl's orientation, A = W "
                       "1024 x 22 limbs (from_float at 0.45 of W/0.02), B = X^T 22 x 64 limbs "
                       "(quantized at 0.5, column-packed), C 1024 x 64 fp32, alpha 1 beta 0",
           "us": d["ms"] * 1e3, "timed_launches": d["timed_launches"],
           "limb_products_per_s": products / (d["ms"] * 1e-3), "limb_products": products,
           "timing": spread_us(d)}
    if with_cpu:
        import numpy as np

        r, kind = _reference_lib()
        a_np, b_np = A[0].cpu().numpy(), B.cpu().numpy()
        times = []
        for _ in range(3):
            c0 = np.zeros((M, N), np.float32)
            t0 = time.perf_counter()
            if r is not None:
                r.gemm_ternary(a_np, b_np, c0, M, N, kl * 48)
            else:
                import oracle

                oracle.gemm_limb(a_np, b_np, c0, M, N, kl * 48)
            times.append(time.perf_counter() - t0)
            if sum(times) > cpu_budget:
                break
        sec = float(np.median(times))
        what = (f"the compiled reference gemm_ternary_cpu_impl ({r.variant}, SIMD "
                f"{r.simd_path()})" if r is not None else
                "the oracle's C restatement of gemm_ternary_cpu_impl")
        out["cpu_baseline"] = {
            "value": products / sec, "unit": "limb products/s", "cores": 1, "kind": kind,
            "sample": f"{what} on the whole config-1 product ({products} limb products), "
                      f"median of {len(times)}: {sec:.2f} s"}
    log(f"limb GEMM config 1: {out['us']:.1f} us, "
        f"{out['limb_products_per_s'] / 1e9:.2f} G limb products/s")
    del A, B, C, x
    torch.cuda.empty_cache()
    return out


def run_backward(torch, ops, lib, dev) -> list:
    """Backward of the Llama gate layer (14336 x 4096): the transposed limbs T^T
    (t81_hip_transpose_packed, graph-timed over rotating weight copies), then dx = dy T as
    the forward product at M = 512 and 2048."""
    rows = []
    k, n = 4096, 14336
    wb = make_weights(torch, ops, lib, n, k, 4, dev, seed=6)
    ms = time_graph(torch, lambda w: ops.transpose_packed(w, n, k), wb, 64, 8)
    tbytes = 16 * n * ((k + 47) // 48) + 16 * k * ((n + 47) // 48)
    gbs = tbytes / (ms * 1e-3) / 1e9
    rows.append({"shape": "transpose_packed llama.gate 14336x4096", "us": ms * 1e3, "GBps": gbs,
                 "frac_hbm": gbs / HBM_PEAK_GBPS})
    log(f"transpose_packed 14336x4096: {ms * 1e3:7.2f} us  {gbs:7.0f} GB/s")
    wt = [ops.transpose_packed(w, n, k) for w in wb[:2]]
    del wb
    for m in (512, 2048):
        dy = torch.randn((m, n), device=dev).to(torch.bfloat16)
        dx = torch.empty((m, k), device=dev)
        ms = time_graph(torch, lambda w: ops.ternary_matmul(dy, w, n, c=dx), wt, 8, 2)
        tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        rows.append({"shape": "backward dx = dy T, llama.gate", "M": m, "K": n, "N": k,
                     "us": ms * 1e3, "TFLOPs": tf, "frac_mfma": tf / BF16_PEAK_TFLOPS})
        log(f"backward dx=dyT llama.gate M={m:5d}: {ms * 1e3:8.1f} us  {tf:7.1f} TFLOP/s")
        del dy, dx
    del wt
    torch.cuda.empty_cache()
    return rows


def run_sweep(torch, ops, lib, dev) -> list:
    """Decode GEMV (config 3 + the Llama gate/down shapes) and prefill GEMM (config 4)."""
    rows = []
    decode = [("phi3.qkv", 3072, 9216), ("phi3.o", 3072, 3072), ("phi3.gate_up", 3072, 16384),
              ("phi3.down", 8192, 3072), ("llama.gate", 4096, 14336), ("llama.down", 14336, 4096)]
    for name, k, n in decode:
        wbytes = 16 * n * ((k + 47) // 48)
        copies = max(4, -(-2 * MALL_BYTES // wbytes) + 2)
        wb = make_weights(torch, ops, lib, n, k, copies, dev, seed=3)
        for m in (1, 4, 16):
            x = torch.randn((m, k), device=dev).to(torch.bfloat16)
            out = torch.empty((m, n), device=dev)
            ms = time_graph(torch, lambda w: ops.ternary_matmul(x, w, k, c=out), wb, 512, 32)
            gbs = gemv_bytes(m, n, k) / (ms * 1e-3) / 1e9
            rows.append({"shape": name, "M": m, "K": k, "N": n, "us": ms * 1e3, "GBps": gbs,
                         "frac_hbm": gbs / HBM_PEAK_GBPS})
            log(f"gemv {name:14s} M={m:2d} {k:5d}->{n:5d}: {ms * 1e3:7.2f} us  {gbs:7.0f} GB/s")
        del wb
        torch.cuda.empty_cache()
    # decode straight from GGUF TQ2_0 payloads (66 bytes per 256 weights)
    from t81lib_amd import gguf
    for name, k, n in [("llama.gate", 4096, 14336), ("llama.down", 14336, 4096),
                       ("phi3.gate_up", 3072, 16384)]:
        pbytes = n * gguf.row_bytes(k, "TQ2_0")
        copies = max(4, -(-2 * MALL_BYTES // pbytes) + 2)
        g = torch.Generator(dev).manual_seed(5)
        wb = [gguf.quantize_tensor(torch.randn((n, k), generator=g, device=dev), "TQ2_0", 0.45)
              for _ in range(copies)]
        for m in (1, 4):
            x = torch.randn((m, k), device=dev).to(torch.bfloat16)
            out = torch.empty((m, n), device=dev)
            ms = time_graph(torch, lambda w: gguf.tq2_matmul(x, w, k, c=out), wb, 512, 32)
            nbytes = pbytes + 2 * m * k + 4 * m * n
            gbs = nbytes / (ms * 1e-3) / 1e9
            rows.append({"shape": name, "format": "TQ2_0", "M": m, "K": k, "N": n,
                         "us": ms * 1e3, "GBps": gbs, "frac_hbm": gbs / HBM_PEAK_GBPS})
            log(f"tq2  {name:14s} M={m:2d} {k:5d}->{n:5d}: {ms * 1e3:7.2f} us  {gbs:7.0f} GB/s")
        del wb
        torch.cuda.empty_cache()
    # the reference's literal matmul_input (config 1: W 1024 x 1024, X 64 x 1024): quantize
    # 0.5 + column pack + limb GEMM fused, against pack_cols then gemm_limb
    wr = make_weights(torch, ops, lib, 1024, 1024, 2, dev, seed=7)
    xr = torch.randn((64, 1024), device=dev)
    cr = torch.zeros((1024, 64), device=dev)
    products = 1024 * 64 * ((1024 + 47) // 48)
    ms = time_graph(torch, lambda w: ops.matmul_input_reference(w, xr, 0.5, c=cr), wr, 16, 2)
    rows.append({"shape": "matmul_input reference_limb fused, config 1", "us": ms * 1e3,
                 "limb_products_per_s": products / (ms * 1e-3)})
    log(f"reference matmul_input fused (config 1): {ms * 1e3:8.1f} us  "
        f"{products / (ms * 1e-3) / 1e9:6.2f} G limb products/s")
    ms2 = time_graph(torch, lambda w: ops.gemm_limb(w, ops.pack_cols(xr, 0.5, lib.THR_TORCH), cr,
                                                     1024, 64, 1024 // 48 * 48 + 48), wr, 16, 2)
    rows.append({"shape": "matmul_input reference_limb two kernels, config 1", "us": ms2 * 1e3,
                 "limb_products_per_s": products / (ms2 * 1e-3)})
    log(f"reference matmul_input pack_cols + gemm_limb: {ms2 * 1e3:8.1f} us")
    del wr, xr, cr
    rows.extend(run_backward(torch, ops, lib, dev))
    # TQ2_0 / TQ1_0 codecs over an 8192 x 3072 float32 matrix
    src = [torch.randn((8192, 3072), device=dev) for _ in range(4)]
    for quant in ("TQ2_0", "TQ1_0"):
        ms = time_graph(torch, lambda w: gguf.quantize_tensor(w, quant, 0.45), src, 64, 8)
        nbytes = 4 * 8192 * 3072 + 8192 * gguf.row_bytes(3072, quant)
        gbs = nbytes / (ms * 1e-3) / 1e9
        rows.append({"shape": f"{quant} quantize 8192x3072", "us": ms * 1e3, "GBps": gbs,
                     "frac_hbm": gbs / HBM_PEAK_GBPS})
        log(f"{quant} quantize 8192x3072: {ms * 1e3:7.2f} us  {gbs:7.0f} GB/s")
        payloads = [gguf.quantize_tensor(w, quant, 0.45) for w in src]
        ms = time_graph(torch, lambda p: gguf.dequantize_tensor(p, (8192, 3072), quant),
                        payloads, 64, 8)
        gbs = nbytes / (ms * 1e-3) / 1e9
        rows.append({"shape": f"{quant} dequantize 8192x3072", "us": ms * 1e3, "GBps": gbs,
                     "frac_hbm": gbs / HBM_PEAK_GBPS})
        log(f"{quant} dequantize 8192x3072: {ms * 1e3:7.2f} us  {gbs:7.0f} GB/s")
        del payloads
    del src
    torch.cuda.empty_cache()
    rows += run_spmm(torch, dev)
    prefill = [("llama.qkv", 4096, 6144), ("llama.gate_up", 4096, 28672),
               ("llama.down", 14336, 4096)]
    for name, k, n in prefill:
        wb = make_weights(torch, ops, lib, n, k, 2, dev, seed=4)
        for m in (512, 2048, 8192):
            x = torch.randn((m, k), device=dev).to(torch.bfloat16)
            out = torch.empty((m, n), device=dev)
            ms = time_graph(torch, lambda w: ops.ternary_matmul(x, w, k, c=out), wb, 8, 2)
            tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
            rows.append({"shape": name, "M": m, "K": k, "N": n, "us": ms * 1e3, "TFLOPs": tf,
                         "frac_mfma": tf / BF16_PEAK_TFLOPS})
            log(f"gemm {name:14s} M={m:5d} {k:5d}->{n:5d}: {ms * 1e3:8.1f} us  {tf:7.1f} TFLOP/s")
            del x, out
        del wb
        torch.cuda.empty_cache()
    return rows


# ------------------------------------------------------------------ profiles --
# Summaries of rocprofv3 output (CSV format) for profiles/.  No GPU needed.

TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_decode_llama_gate_m1_traffic.txt")


def _read_csv(path: str) -> list:
    import csv
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def _find(d: str, suffix: str) -> str:
    for name in sorted(os.listdir(d)):
        if name.endswith(suffix):
            return os.path.join(d, name)
    raise FileNotFoundError(f"no *{suffix} in {d}")


def summarize_trace(d: str, cmd: str, top: int = 8) -> str:
    """Kernel table of a `rocprofv3 --kernel-trace --stats --output-format csv` run."""
    rows = _read_csv(_find(d, "kernel_stats.csv"))
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    out = [f"command: {cmd}", "",
           f"{'calls':>6} {'avg_us':>9} {'min_us':>9} {'max_us':>9} {'total_%':>8}  kernel"]
    for r in rows[:top]:
        out.append(f"{int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:9.2f} "
                   f"{float(r['MinNs']) / 1e3:9.2f} {float(r['MaxNs']) / 1e3:9.2f} "
                   f"{float(r['Percentage']):8.2f}  {r['Name'][:110]}")
    return "\n".join(out) + "\n"


def summarize_trace_by_grid(d: str, kernel_sub: str, cmd: str, runs: bool = False,
                            gap_ms: float = 1.0) -> str:
    """Per-dispatch table of a `rocprofv3 --kernel-trace --output-format csv` run, grouped by
    kernel and launch shape (grid x workgroup size, which tells apart the shapes one kernel
    instance serves), for the kernels whose name contains kernel_sub, in first-launch order.
    runs: one row per run of consecutive such dispatches with the same key (in start order),
    so that two shapes with one launch shape, timed one after the other, stay apart; a run
    also ends where the GPU ran none of these kernels for more than gap_ms (the host setting
    up the next timed case) or where a dispatch takes more than 1.6 x or less than 1 / 1.6 x
    the run's mean so far (the next shape on the same launch shape); two keys whose
    dispatches strictly alternate (two launches per call, as float32 activations' two
    planes) keep one row each for the stretch they alternate over."""
    rows = [r for r in _read_csv(_find(d, "kernel_trace.csv")) if kernel_sub in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    groups: list = []
    index: dict = {}
    keys: list = []
    last_end = None
    for r in rows:
        key = (r["Kernel_Name"], int(r["Grid_Size_X"]), int(r["Workgroup_Size_X"]))
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        gap = last_end is not None and int(r["Start_Timestamp"]) - last_end > gap_ms * 1e6
        last_end = int(r["End_Timestamp"])
        if gap:
            keys = []
        keys.append(key)
        if runs:
            def near(ts):
                mean = sum(ts) / len(ts)
                return mean / 1.6 <= us <= 1.6 * mean
            if groups and groups[-1][0] == key and not gap and near(groups[-1][1]):
                groups[-1][1].append(us)
            elif (len(groups) >= 2 and groups[-2][0] == key and len(keys) >= 3 and
                  keys[-3] == key and near(groups[-2][1])):
                groups[-2][1].append(us)
            else:
                groups.append((key, [us]))
        else:
            if key not in index:
                index[key] = len(groups)
                groups.append((key, []))
            groups[index[key]][1].append(us)
    out = [f"command: {cmd}", "",
           f"{'calls':>6} {'avg_us':>8} {'min_us':>8} {'max_us':>8} {'workgroups':>10} "
           f"{'threads':>7}  kernel"]
    for (name, grid, wg), ts in groups:
        out.append(f"{len(ts):6d} {sum(ts) / len(ts):8.2f} {min(ts):8.2f} {max(ts):8.2f} "
                   f"{grid // wg:10d} {wg:7d}  {name[:100]}")
    return "\n".join(out) + "\n"


def _counter_median(d: str, kernel_sub: str, counter: str) -> tuple:
    import statistics
    vals = [float(r["Counter_Value"]) for r in _read_csv(_find(d, "counter_collection.csv"))
            if kernel_sub in r["Kernel_Name"] and r["Counter_Name"] == counter]
    if not vals:
        raise ValueError(f"no {counter} rows for '{kernel_sub}' in {d}")
    return statistics.median(vals), len(vals)


def summarize_counters(d: str, kernel_sub: str, cmd: str) -> str:
    """Median per dispatch of every counter a `rocprofv3 --pmc` run collected for the kernels
    whose name contains `kernel_sub`.  When the MFMA busy cycles and the GPU busy cycles are
    both there: MFMA busy per SIMD over the busy time (GRBM_GUI_ACTIVE counts the shader
    clock of each of the 8 XCDs; 1024 SIMDs)."""
    import statistics
    rows = [r for r in _read_csv(_find(d, "counter_collection.csv")) if kernel_sub in r["Kernel_Name"]]
    if not rows:
        raise ValueError(f"no rows for '{kernel_sub}' in {d}")
    by: dict = {}
    for r in rows:
        by.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    names = sorted({r["Kernel_Name"][:110] for r in rows})
    out = [f"command: {cmd}", "", "kernels: " + "; ".join(names), ""]
    med = {k: statistics.median(v) for k, v in by.items()}
    for k in sorted(med):
        out.append(f"{k:28s} {med[k]:18.0f}   (median of {len(by[k])} dispatches)")
    if "SQ_VALU_MFMA_BUSY_CYCLES" in med and "GRBM_GUI_ACTIVE" in med:
        per_xcd = med["GRBM_GUI_ACTIVE"] / 8.0
        busy = med["SQ_VALU_MFMA_BUSY_CYCLES"] / 1024.0
        out += ["", f"MFMA busy per SIMD: {busy:.0f} of {per_xcd:.0f} busy cycles = "
                    f"{100.0 * busy / per_xcd:.1f} %"]
    return "\n".join(out) + "\n"


def summarize_traffic(kernel: str, kfetch: str, kwrite: str, cfetch: str, cwrite: str,
                      copy_bytes: int, algo_bytes: int, cmds: list) -> str:
    """HBM bytes per launch of `kernel` from FETCH_SIZE / WRITE_SIZE runs, each scaled by
    what the same counter reads for a plain copy (torch.neg) of `copy_bytes` each way."""
    cf, _ = _counter_median(cfetch, "elementwise_kernel", "FETCH_SIZE")
    cw, _ = _counter_median(cwrite, "elementwise_kernel", "WRITE_SIZE")
    kf, nf = _counter_median(kfetch, kernel, "FETCH_SIZE")
    kw, nw = _counter_median(kwrite, kernel, "WRITE_SIZE")
    f_scale = copy_bytes / (cf * 1024.0)
    w_scale = copy_bytes / (cw * 1024.0)
    fetch = kf * 1024.0 * f_scale
    write = kw * 1024.0 * w_scale
    out = ["commands:"] + [f"  {c}" for c in cmds] + [
        "",
        f"kernel: {kernel}",
        f"copy calibration: torch.neg over {copy_bytes} B each way; FETCH_SIZE reads "
        f"{cf:.1f} KiB (scale {f_scale:.4f}), WRITE_SIZE reads {cw:.1f} KiB (scale {w_scale:.4f})",
        f"kernel FETCH_SIZE median {kf:.1f} KiB over {nf} dispatches -> {fetch:.0f} B",
        f"kernel WRITE_SIZE median {kw:.1f} KiB over {nw} dispatches -> {write:.0f} B",
        f"algorithmic bytes per launch: {algo_bytes}",
        f"hbm_bytes_per_launch: {int(round(fetch + write))}",
        f"traffic / algorithmic: {(fetch + write) / algo_bytes:.4f}",
    ]
    return "\n".join(out) + "\n"


def read_traffic(path: str = TRAFFIC_FILE):
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it: model name, vendor, family / model /
    stepping numbers and the SIMD extensions the reference path can use."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" not in line:
                    if fields:
                        break          # the first processor's block is enough
                    continue
                key, val = (p.strip() for p in line.split(":", 1))
                fields.setdefault(key, val)
    except OSError:
        return "unknown"
    flags = fields.get("flags", "").split()
    simd = [f for f in ("avx2", "avx512f", "avx512bw", "avx512_vnni", "avx512_bf16") if f in flags]
    return (f"{fields.get('model name', 'unknown')} ({fields.get('vendor_id', '?')}, family "
            f"{fields.get('cpu family', '?')} model {fields.get('model', '?')} stepping "
            f"{fields.get('stepping', '?')}, {fields.get('cache size', '?')} cache, "
            f"{' '.join(simd) or 'no avx2'})")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="seconds of single-core reference CPU work for the baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["gemv", "gemm", "pack", "copy", "read", "spmm", "launch",
                                       "stack", "decode", "backward", "prefill", "limb",
                                       "pack3072", "gemv_valu", "aux"],
                    default=None,
                    help="time one kernel only (for profiling runs); 'copy' times a plain "
                         "elementwise copy of the GEMV weight size, the calibration kernel "
                         "for the HBM byte counters; 'read' a plain reduction over the GEMV "
                         "weight copies (the read floor); 'launch' a one-element fill, the "
                         "per-launch floor of a graph of back-to-back kernels; 'stack' runs "
                         "config 5, the 32-layer decoder, prefill + greedy decode tokens/s; "
                         "'backward' the transposed limbs and dx = dy T of the Llama gate layer")
    ap.add_argument("--decode-case", nargs=3, type=int, metavar=("K", "N", "M"), default=None,
                    help="with --only decode: time this one shape and token count only")
    ap.add_argument("--no-stack", action="store_true",
                    help="skip config 5 (the decoder stack) in the default run")
    ap.add_argument("--sweep", action="store_true",
                    help="also time the config-3/4 shapes and print a table on stderr")
    ap.add_argument("--summarize-trace", metavar="DIR",
                    help="print the kernel table of a rocprofv3 csv --stats run and exit")
    ap.add_argument("--summarize-trace-by-grid", nargs=2, metavar=("DIR", "KERNEL"),
                    help="print the dispatches of a rocprofv3 csv --kernel-trace run grouped "
                         "by kernel and launch shape, for kernels whose name contains KERNEL")
    ap.add_argument("--runs", action="store_true",
                    help="with --summarize-trace-by-grid: one row per run of consecutive "
                         "dispatches instead of one per launch shape")
    ap.add_argument("--summarize-counters", nargs=2, metavar=("DIR", "KERNEL"),
                    help="print the median counters of a rocprofv3 csv --pmc run for the "
                         "kernels whose name contains KERNEL, and exit")
    ap.add_argument("--summarize-traffic", nargs=4, metavar=("KFETCH", "KWRITE", "CFETCH", "CWRITE"),
                    help="print calibrated HBM bytes per GEMV launch from rocprofv3 --pmc "
                         "FETCH_SIZE / WRITE_SIZE runs of the GEMV and of the copy, and exit")
    ap.add_argument("--traffic-kernel", choices=["gemv", "pack"], default="gemv",
                    help="with --summarize-traffic: the K2 headline launch (gemv) or K1 on "
                         "8192 x 3072 (pack, from --only pack runs)")
    ap.add_argument("--cmd", action="append", default=[],
                    help="command line(s) that produced the profile, for the summary")
    args = ap.parse_args()
    if args.summarize_trace:
        sys.stdout.write(summarize_trace(args.summarize_trace, " | ".join(args.cmd)))
        return 0
    if args.summarize_trace_by_grid:
        sys.stdout.write(summarize_trace_by_grid(*args.summarize_trace_by_grid,
                                                 " | ".join(args.cmd), runs=args.runs))
        return 0
    if args.summarize_counters:
        sys.stdout.write(summarize_counters(*args.summarize_counters, " | ".join(args.cmd)))
        return 0
    if args.summarize_traffic:
        K, N = 4096, 14336
        wb = 16 * N * ((K + 47) // 48)
        if args.traffic_kernel == "pack":
            kernel, algo = "quantize_pack_rows_kernel", 4 * 8192 * 3072 + 16 * 8192 * 64
        else:
            kernel, algo = "gemv", gemv_bytes(1, N, K)
        sys.stdout.write(summarize_traffic(kernel, *args.summarize_traffic, copy_bytes=wb,
                                           algo_bytes=algo, cmds=args.cmd))
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the packed-ternary path is a single-GPU kernel set "
              "(multi-GPU sharding is a design note only); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    from t81lib_amd import _lib, ops

    if not torch.cuda.is_available() or not _lib.available():
        print("bench.py needs a gfx950 GPU and libt81_hip.so", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    only = args.only
    threads = cpu_threads()

    # ---------------------------------------------------------- K2 decode GEMV --
    M, K, N = 1, 4096, 14336
    wbytes = 16 * N * ((K + 47) // 48)
    copies = max(8, -(-2 * MALL_BYTES // wbytes) + 4)
    gemv = None
    floors: dict = {}
    if only in (None, "gemv", "read", "copy", "launch"):
        log(f"GEMV {K}->{N} M={M}: {copies} weight copies of {wbytes / 1e6:.1f} MB, "
            f"{args.steps} timed launches issued one by one through the C ABI")
        wbufs = make_weights(torch, ops, _lib, N, K, copies, dev, seed=1)
        x = torch.randn((M, K), device=dev).to(torch.bfloat16)
        if only in (None, "gemv"):
            out = torch.empty((M, N), device=dev)
            # the C ABI entry point itself, called once per launch (the host issues a call in
            # ~3.5 us, the GPU runs one in ~6.5 us, so the queue never drains)
            abi = _lib.lib().t81_hip_ternary_matmul_kernel
            wptrs = [wb.data_ptr() for wb in wbufs]
            xptr, optr = x.data_ptr(), out.data_ptr()

            def launch(i, sh, abi=abi, wptrs=wptrs, xptr=xptr, optr=optr, dt=_lib.DTYPE_BF16):
                rc = abi(2, xptr, dt, wptrs[i], optr, M, N, K, 1.0, 0.0, None, sh)
                if rc != 0:
                    _lib.check(rc)

            gemv = time_eager(torch, launch, len(wbufs), args.steps, args.warmup)
            gemv["sha256"] = sha256_tensors(torch, wbufs[0], x)
            log(f"GEMV {gemv['ms'] * 1e3:.2f} us/call over {args.steps} calls "
                f"(median {gemv['median_ms'] * 1e3:.2f}, p10 {gemv['p10_ms'] * 1e3:.2f}, "
                f"p90 {gemv['p90_ms'] * 1e3:.2f})")
        if only in (None, "read"):
            # the read floor: a plain coalesced streaming read of the same weight copies
            # (csrc/floors.hip), best over grid sizes and loads in flight per thread
            import ctypes

            flib = ctypes.CDLL(os.path.join(ROOT, "t81lib_amd", "libt81_floors.so"))
            flib.t81_floor_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                            ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
            sink = torch.empty(8192, dtype=torch.int32, device=dev)
            best = None
            for unroll in (1, 4, 8):
                for blocks in (256, 512, 1024, 2048, 4096):
                    def rd(wb, blocks=blocks, unroll=unroll):
                        rc = flib.t81_floor_read(wb.data_ptr(), wbytes, sink.data_ptr(), blocks,
                                                 unroll, torch.cuda.current_stream().cuda_stream)
                        if rc != 0:
                            raise RuntimeError(f"t81_floor_read failed ({rc})")
                    r = time_graph(torch, rd, wbufs, max(args.steps, 256), 32, dist=True)
                    if best is None or r["median_ms"] < best[2]["median_ms"]:
                        best = (blocks, unroll, r)
            blocks, unroll, r = best
            floors["read"] = {"workload": f"plain coalesced read of one {wbytes}-byte weight "
                                          f"copy (16-byte loads, {blocks} workgroups of 256, "
                                          f"{unroll} loads in flight per thread; best of "
                                          f"256-4096 workgroups x 1, 4, 8 loads), "
                                          f"{copies} rotating copies",
                              "us": r["median_ms"] * 1e3,
                              "GBps": wbytes / (r["median_ms"] * 1e-3) / 1e9, **spread_us(r)}
            log(f"read floor {floors['read']['us']:.2f} us/launch, "
                f"{floors['read']['GBps']:.0f} GB/s ({blocks} workgroups, {unroll} in flight)")
        if only in (None, "copy"):
            # counter calibration and the measured copy bandwidth (read + write)
            elems = wbytes // 4
            ccopies = max(4, -(-2 * MALL_BYTES // wbytes) + 2)
            csrc = [torch.randn(elems, device=dev) for _ in range(ccopies)]
            cdst = torch.empty(elems, device=dev)
            cp = time_graph(torch, lambda t: torch.neg(t, out=cdst), csrc,  # noqa: E731
                            max(args.steps, 256), 32, dist=True)
            floors["copy"] = {"workload": f"torch.neg fp32, {elems} elements: reads and writes "
                                          f"{4 * elems} bytes per launch",
                              "bytes_read": 4 * elems, "bytes_written": 4 * elems,
                              "us": cp["median_ms"] * 1e3,
                              "GBps": 8 * elems / (cp["median_ms"] * 1e-3) / 1e9,
                              **spread_us(cp)}
            del csrc, cdst
            log(f"copy {floors['copy']['us']:.2f} us/launch, {floors['copy']['GBps']:.0f} GB/s")
        if only in (None, "launch"):
            tiny = [torch.zeros(1, device=dev) for _ in range(32)]
            lf = time_graph(torch, lambda t: t.fill_(1.0), tiny, max(args.steps, 256), 32,  # noqa
                            dist=True)
            floors["launch"] = {"workload": "graph of one-element torch fill_ launches",
                                "us": lf["median_ms"] * 1e3, **spread_us(lf)}
            log(f"launch floor {floors['launch']['us']:.2f} us/launch")
        del wbufs
        torch.cuda.empty_cache()

    # --------------------------------------------------------- K3 prefill GEMM --
    GM, GK, GN = 2048, 4096, 28672
    gemm = None
    if only in (None, "gemm"):
        log(f"GEMM M={GM} {GK}->{GN}")
        gw = make_weights(torch, ops, _lib, GN, GK, 2, dev, seed=2)
        gx = torch.randn((GM, GK), device=dev).to(torch.bfloat16)
        gout = torch.empty((GM, GN), device=dev)
        # exactly 100 timed launches (and >= 50 ms of spread samples) whatever --steps is,
        # after 20 untimed ones that bring the clocks to their loaded state; issued one by
        # one through the C ABI, as the headline leg (this shape needs no workspace)
        assert _lib.lib().t81_hip_ternary_matmul_workspace_size(GM, GN, GK, _lib.DTYPE_BF16) == 0
        gemm = time_eager(torch, abi_launch(_lib, gx, _lib.DTYPE_BF16, gw, gout, GM, GN, GK),
                          len(gw), 100, 20, ahead=4)
        gemm["sha256"] = sha256_tensors(torch, gw[0], gx)
        del gw, gx, gout
        torch.cuda.empty_cache()
        log(f"GEMM {gemm['ms']:.3f} ms/call over 100 calls (median {gemm['median_ms']:.3f})")

    # ----------------------------------------- K3 prefill GEMM, int8 activations --
    gemm_i8 = None
    if only in (None, "gemm"):
        log(f"GEMM int8 M={GM} {GK}->{GN}")
        gw = make_weights(torch, ops, _lib, GN, GK, 2, dev, seed=2)
        gx8 = torch.randint(-128, 128, (GM, GK), device=dev, dtype=torch.int8)
        gout8 = torch.empty((GM, GN), device=dev, dtype=torch.int32)
        assert _lib.lib().t81_hip_ternary_matmul_workspace_size(GM, GN, GK, _lib.DTYPE_I8) == 0
        gemm_i8 = time_eager(torch, abi_launch(_lib, gx8, _lib.DTYPE_I8, gw, gout8, GM, GN, GK),
                             len(gw), 100, 20, ahead=4)
        gemm_i8["sha256"] = sha256_tensors(torch, gw[0], gx8)
        del gw, gx8, gout8
        torch.cuda.empty_cache()
        log(f"GEMM int8 {gemm_i8['ms']:.3f} ms/call over 100 calls "
            f"(median {gemm_i8['median_ms']:.3f})")

    # ------------------------------------------------------------- K1 pack --
    # config 2: W ~ N(0, 0.02) with 1 % outliers x 10, threshold 0.45 (C++ form)
    PR, PC = 8192, 3072
    pack = None
    pack3072 = None

    def time_pack(rows, cols, which):
        pbytes = 4 * rows * cols + 16 * rows * ((cols + 47) // 48)
        pcopies = max(4, -(-2 * MALL_BYTES // pbytes) + 2)
        gen = torch.Generator(dev).manual_seed(rows + cols)
        srcs = []
        for _ in range(pcopies):
            w = torch.randn((rows, cols), device=dev, generator=gen) * 0.02
            w = torch.where(torch.rand((rows, cols), device=dev, generator=gen) < 0.01, w * 10, w)
            srcs.append(w)
        pout = torch.empty((rows, (cols + 47) // 48, 16), dtype=torch.uint8, device=dev)
        qp = _lib.lib().t81_hip_quantize_pack
        sptrs = [t.data_ptr() for t in srcs]
        outp = pout.data_ptr()

        def plaunch(i, sh):
            rc = qp(sptrs[i], _lib.DTYPE_F32, outp, rows, cols, 0.45, _lib.THR_CPP, sh)
            if rc != 0:
                _lib.check(rc)

        # launches issued one by one through the C ABI (host ~3.5 us per call, the kernel
        # ~9-20 us), as the other legs
        r = time_eager(torch, plaunch, len(srcs), max(128, args.steps // 8), 8)
        r["sha256"] = sha256_tensors(torch, srcs[0])
        del srcs
        torch.cuda.empty_cache()
        log(f"pack {rows}x{cols} ({which}) {r['ms'] * 1e3:.2f} us/call "
            f"(median {r['median_ms'] * 1e3:.2f})")
        return r

    if only in (None, "pack"):
        pack = time_pack(PR, PC, "8192x3072")
    if only in (None, "pack3072"):
        pack3072 = time_pack(3072, 3072, "3072x3072")

    # ------------------------------------------------------------ CPU baselines --
    cpu = None
    if not args.no_cpu and only is None:
        budget = args.cpu_budget
        log(f"CPU baselines: reference gemm_ternary and pack, 1 and {threads} threads")
        g1, d1 = cpu_reference_gemv(N, K, 0.35 * budget, 1)
        ga, da = cpu_reference_gemv(N, K, 0.1 * budget, threads)
        host = f"host {cpu_model()}, nproc {os.cpu_count()}"
        cpu = {
            "value": g1, "unit": "GB/s", "cores": 1, "kind": d1["kind"],
            "sample": (f"reference gemm_ternary_cpu_impl ({d1['variant']}, SIMD {d1['simd']}) "
                       f"on {d1['rows']} of {N} weight rows x {(K + 47) // 48} limbs x 1 packed "
                       f"activation column = {d1['limb_products']} limb products in "
                       f"{d1['seconds']:.2f} s; GB/s of packed weights streamed; {host}"),
            "all_cores": {"value": ga, "unit": "GB/s", "cores": threads, "kind": da["kind"],
                          "sample": f"same kernel over {da['rows']} rows in 16-row blocks on "
                                    f"{threads} threads, {da['seconds']:.2f} s"},
        }
        if gemm is not None:
            t1, e1 = cpu_reference_gemm(GM, GN, GK, 256, 64, 0.3 * budget, 1)
            ta, ea = cpu_reference_gemm(GM, GN, GK, 1024, 64, 0.1 * budget, threads)
            gemm["cpu_baseline"] = {
                "value": t1, "unit": "TFLOP/s-equivalent", "cores": 1, "kind": e1["kind"],
                "sample": (f"reference gemm_ternary_cpu_impl on {e1['rows']} weight rows x 64 "
                           f"packed activation columns x {(GK + 47) // 48} limbs "
                           f"({e1['limb_products']} limb products, {e1['seconds']:.2f} s), "
                           f"extrapolated linearly in M*N*L to {GM}x{GN}x{GK}: "
                           f"{e1['extrapolated_full_s']:.0f} s; 2*M*N*K flops"),
                "all_cores": {"value": ta, "unit": "TFLOP/s-equivalent", "cores": threads,
                              "kind": ea["kind"],
                              "sample": f"{ea['rows']} rows x 64 columns on {threads} threads, "
                                        f"extrapolated: {ea['extrapolated_full_s']:.0f} s"},
            }
        if pack is not None:
            p1, s1 = cpu_pack(PR, PC, 1)
            pa, sa = cpu_pack(PR, PC, threads)
            pack["cpu_baseline"] = {
                "value": p1, "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": (f"the oracle's C restatement of pack_dense_matrix "
                           f"(python/bindings.cpp:497-515) on the full {PR}x{PC} float32 matrix, "
                           f"median of 3: {s1 * 1e3:.1f} ms"),
                "all_cores": {"value": pa, "unit": "GB/s", "cores": threads, "kind": "port",
                              "sample": f"row blocks on {threads} threads, {sa * 1e3:.1f} ms"},
            }

    limb = run_limb(torch, ops, _lib, dev, 0.25 * args.cpu_budget, not args.no_cpu and only is None) \
        if only in (None, "limb") else None
    prefill = run_prefill(torch, ops, _lib, dev) if only in (None, "prefill") else None
    gemv_valu = run_gemv_valu(torch, ops, _lib, dev) if only in (None, "gemv_valu") else None
    decode = run_decode(torch, ops, _lib, dev, args.decode_case) \
        if only in (None, "decode") else None
    sweep = run_sweep(torch, ops, _lib, dev) if args.sweep else None
    spmm = run_spmm(torch, dev) if only == "spmm" else None
    aux = run_aux(torch, ops, _lib, dev) if only == "aux" else None
    backward = run_backward(torch, ops, _lib, dev) if only == "backward" else None
    stack = run_stack(torch, dev) if only == "stack" or (only is None and not args.no_stack) \
        else None

    gemv_ms = gemv["ms"] if gemv else None
    gbytes = gemv_bytes(M, N, K)
    line: dict = {
        "metric": METRIC,
        "value": (gbytes / (gemv_ms * 1e-3) / 1e9) if gemv_ms else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": gemv_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: W ~ N(0,1) (the effective W/0.02) ternarized at 0.45, x ~ N(0,1) bf16",
        "config": {"workload": f"decode GEMV K2, {K}->{N} (Llama-3-8B gate), M={M}, bf16 x, "
                               f"fp32 out, alpha=1 beta=0, {copies} rotating weight copies",
                   "M": M, "K": K, "N": N, "parallelism": "none (1 GPU)"},
    }
    if gemv_ms:
        achieved = gbytes / (gemv_ms * 1e-3) / 1e9
        line["roofline"] = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS,
                            "unit": "GB/s", "frac": achieved / HBM_PEAK_GBPS,
                            "traffic": read_traffic()}
        if "copy" in floors:
            line["roofline"]["measured_copy_GBps"] = floors["copy"]["GBps"]
            line["roofline"]["frac_of_measured_copy"] = achieved / floors["copy"]["GBps"]
        line["timing"] = {**spread_us(gemv), "timed_launches": gemv["timed_launches"],
                          "method": "launches issued one by one through the C ABI "
                                    "(t81_hip_ternary_matmul_kernel) behind 64 untimed ones, "
                                    "HIP events on the launch stream around the timed ones"}
        line["tokens_per_s_equiv"] = M / (gemv_ms * 1e-3)
        line["inputs_sha256"] = gemv["sha256"]
    if cpu:
        line["cpu_baseline"] = cpu
    if gemm:
        flops = 2.0 * GM * GN * GK
        tflops = flops / (gemm["ms"] * 1e-3) / 1e12
        line["gemm"] = {
            "workload": f"prefill GEMM K3, M={GM}, {GK}->{GN} (Llama-3-8B gate_up), bf16 x",
            "ms": gemm["ms"], "timed_launches": gemm["timed_launches"], "tflops": tflops,
            "tokens_per_s_equiv": GM / (gemm["ms"] * 1e-3),
            "roofline": {"bound": "mfma", "achieved": tflops, "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": tflops / BF16_PEAK_TFLOPS},
            "timing": spread_us(gemm), "inputs_sha256": gemm["sha256"],
        }
        if "cpu_baseline" in gemm:
            line["gemm"]["cpu_baseline"] = gemm["cpu_baseline"]
    if gemm_i8:
        tops = 2.0 * GM * GN * GK / (gemm_i8["ms"] * 1e-3) / 1e12
        line["gemm_int8"] = {
            "workload": f"prefill GEMM K3, M={GM}, {GK}->{GN} (Llama-3-8B gate_up), int8 x, "
                        f"exact int32 out (integer matrix cores)",
            "ms": gemm_i8["ms"], "timed_launches": gemm_i8["timed_launches"], "tops": tops,
            "roofline": {"bound": "mfma", "achieved": tops, "peak": INT8_PEAK_TOPS,
                         "unit": "TOP/s", "frac": tops / INT8_PEAK_TOPS},
            "timing": spread_us(gemm_i8), "inputs_sha256": gemm_i8["sha256"],
        }
    if pack:
        pbytes = 4 * PR * PC + 16 * PR * ((PC + 47) // 48)
        gbs = pbytes / (pack["ms"] * 1e-3) / 1e9
        line["pack"] = {"workload": f"K1 quantize+pack {PR}x{PC} fp32", "us": pack["ms"] * 1e3,
                        "timed_launches": pack["timed_launches"],
                        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBPS,
                                     "unit": "GB/s", "frac": gbs / HBM_PEAK_GBPS},
                        "timing": spread_us(pack), "inputs_sha256": pack["sha256"]}
        if "cpu_baseline" in pack:
            line["pack"]["cpu_baseline"] = pack["cpu_baseline"]
    if pack3072:
        pbytes3 = 4 * 3072 * 3072 + 16 * 3072 * 64
        gbs3 = pbytes3 / (pack3072["ms"] * 1e-3) / 1e9
        entry = {"workload": "K1 quantize+pack 3072x3072 fp32 (config 2)",
                 "us": pack3072["ms"] * 1e3, "timed_launches": pack3072["timed_launches"],
                 "roofline": {"bound": "hbm", "achieved": gbs3, "peak": HBM_PEAK_GBPS,
                              "unit": "GB/s", "frac": gbs3 / HBM_PEAK_GBPS},
                 "timing": spread_us(pack3072), "inputs_sha256": pack3072["sha256"]}
        if "pack" in line:
            line["pack"]["config2_3072x3072"] = entry
        else:
            line["pack"] = {"config2_3072x3072": entry}
    if limb:
        line["limb"] = limb
    if prefill:
        line["prefill"] = prefill
    if gemv_valu:
        line["gemv_valu_ab"] = gemv_valu
    if floors:
        line["floors"] = floors
    if decode:
        line["decode"] = decode
    if sweep:
        line["sweep"] = sweep
    if spmm:
        line["spmm"] = spmm
    if aux:
        line["aux"] = aux
    if backward:
        line["backward"] = backward
    if stack:
        line["stack"] = stack
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
