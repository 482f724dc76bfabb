#!/usr/bin/env python3
"""Benchmark of the HiF8 static W8A8KV8 hot path on one MI355X.

Headline (``value``): the decode GEMV sweep of BASELINE configs[1] - for
M in {1, 4}, every projection of one 9B-class decoder layer (q 4096x4096,
fused k+v 2048x4096, o 4096x4096, fused gate+up 24576x4096, down 4096x12288)
runs the static W8A8 linear method (hif8_rocm.scheme) with its default
routing: decode-sized inputs through the fused op soft_hif8_static_fused_gemm
(one launch for one row, and for four rows with K <= 4096 and N <= 2048 on
the MFMA-4 GEMV; hif8_static_quant then the code GEMV inside the op
otherwise; outputs equal to the two-stage route).  The reference's
routing (every projection as static quant + soft_hif8_gemm,
HIF8_STATIC_FUSED_SINGLE_ROW=0) is reported beside it.  One step = that sweep over one layer's weights; five
distinct weight copies (966 MB) are rotated so the 256 MB Infinity Cache
cannot serve them.  Steps are captured in HIP graphs and replayed, so host
launch overhead is not timed; ~400 untimed replays (the W warm-up steps
included) settle the clock before the K timed steps.

``value`` = algorithmic bytes of the step (weights + activations + scales +
outputs of every quant and GEMV launch) / wall time per step, in GB/s.
Secondary figures (prefill GEMM TFLOP/s, also over weights kept decoded to
bf16 under HIF8_PREFILL_BF16_WEIGHTS=1; static quant GB/s; KV decode
attention; the synthetic end-to-end decode) and a per-kernel table are
reported in the same JSON line.

Synthetic data: bf16 activations ~N(0,1) with a static scale absmax/32768;
weights ~N(0, 0.02) with per-row scales absmax/32768, encoded on the GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
PKG_ROOT = REPO / "gcc-hif8-quantized-from-qwen3.5-9b_amd"
for _p in (str(REPO), str(PKG_ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "HiF8 GEMV GB/s & GEMM TFLOP/s vs MI355X roofline; KV8 decode-attn μs/token"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
HIF8_MAX = 32768.0
LAYER = [("q", 4096, 4096), ("kv", 2048, 4096), ("o", 4096, 4096), ("gate_up", 24576, 4096), ("down", 4096, 12288)]
DECODE_M = (1, 4)
PREFILL_M = (512, 4096)
N_COPIES = 5
ROTATE_BYTES = 768 * 2 ** 20   # weight bytes rotated per per-kernel row (> 3x the 256 MB Infinity Cache)
MIN_TIMED_LAUNCHES = 100        # per-kernel rows: median over at least this many launches
SETTLE_STEPS = 400              # untimed headline replays (warm-up included) before the timed steps
HOST_LIB = PKG_ROOT / "hif8_rocm" / "libhif8_rocm.so"
# KV8 decode attention: 16 query heads, 4 KV heads, head_dim 256, 128-token pages.
KV_HQ, KV_HKV, KV_D, KV_BS = 16, 4, 256, 128
KV_CTX = (512, 4096, 16384)
KV_BATCH = (1, 4)
KV_CALLS_PER_GRAPH = 4
KV_POOL_BYTES = 1_100_000_000   # K + V page pool, > 4x the Infinity Cache


def gemv_bytes(m: int, n: int, k: int) -> int:
    return n * k + m * k + 4 * n + 4 * m + 2 * m * n


def quant_bytes(m: int, k: int) -> int:
    return 3 * m * k + 4 * m + 4


def kv_attention_bytes(lens) -> int:
    """K and V rows of every context token (codes + sidecar), q in, out, block-table entries."""
    pages = sum((n + KV_BS - 1) // KV_BS for n in lens)
    return (sum(lens) * KV_HKV * (KV_D + 4) * 2 + 2 * len(lens) * KV_HQ * KV_D * 2 + 4 * pages)


def kv_write_bytes(tokens: int) -> int:
    """bf16 K and V in, packed K and V rows out, 8-byte slots."""
    return tokens * KV_HKV * (2 * KV_D * 2 + (KV_D + 4) * 2) + 8 * tokens


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Setup:
    def __init__(self, torch, native, device):
        from hif8_rocm.scheme import W8A8HiFloat8StaticLinearMethod

        self.torch, self.native, self.device = torch, native, device
        self.method = W8A8HiFloat8StaticLinearMethod()
        g = torch.Generator(device=device).manual_seed(20261201)
        self.x = {}
        for m in DECODE_M + PREFILL_M:
            for k in sorted({k for _, _, k in LAYER}):
                x = torch.randn(m, k, generator=g, device=device).to(torch.bfloat16)
                s = (x.float().abs().amax() / HIF8_MAX).reshape(1).contiguous()
                self.x[(m, k)] = (x, s)
        self.rot = {}      # name -> rotated weight copies of >= ROTATE_BYTES (per-kernel rows)
        self.weights = []  # [copy][name] -> (codes u8 [N,K], scale f32 [N])
        self.layers = []   # [copy][name] -> module with weight / weight_scale / input_scale
        for _ in range(N_COPIES):
            ws_by_name, mods = {}, {}
            for name, n, k in LAYER:
                w = (torch.randn(n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
                ws = (w.float().abs().amax(dim=1) / HIF8_MAX).contiguous()
                codes, _ = native.static_quant(w, ws)
                del w
                ws_by_name[name] = (codes, ws)
                mod = torch.nn.Module()
                mod.weight = torch.nn.Parameter(codes, requires_grad=False)
                mod.weight_scale = torch.nn.Parameter(ws.reshape(-1, 1).clone(), requires_grad=False)
                mod.input_scale = torch.nn.Parameter(self.x[(1, k)][1].clone(), requires_grad=False)
                self.method.process_weights_after_loading(mod)
                mods[name] = mod
            self.weights.append(ws_by_name)
            self.layers.append(mods)
        torch.cuda.synchronize()


class KVSetup:
    """One page pool of HiF8 K/V (written by the fused write kernel) and, per
    (batch, ctx), several block tables over disjoint random pages, rotated
    between steps so each step reads pages no earlier step touched."""

    def __init__(self, torch, device):
        from hif8_rocm import kv_cache

        self.torch, self.device = torch, device
        page_bytes = KV_BS * KV_HKV * (KV_D + 4) * 2
        self.num_blocks = KV_POOL_BYTES // page_bytes
        layout = kv_cache.Hif8KVCacheLayout(self.num_blocks, KV_BS, KV_HKV, KV_D)
        self.kc, self.vc = layout.allocate(device)
        g = torch.Generator(device=device).manual_seed(4242)
        chunk = 32768
        tokens = self.num_blocks * KV_BS
        self.ks = self.vs = None
        for t0 in range(0, tokens, chunk):
            n = min(chunk, tokens - t0)
            k = torch.randn(n, KV_HKV, KV_D, generator=g, device=device).to(torch.bfloat16)
            v = torch.randn(n, KV_HKV, KV_D, generator=g, device=device).to(torch.bfloat16)
            if self.ks is None:   # static per-head scales from the first chunk: absmax / 32768
                self.ks = (k.float().abs().amax(dim=(0, 2)) / HIF8_MAX).contiguous()
                self.vs = (v.float().abs().amax(dim=(0, 2)) / HIF8_MAX).contiguous()
            slots = torch.arange(t0, t0 + n, device=device, dtype=torch.int64)
            kv_cache.write_kv_cache(k, v, self.kc, self.vc, slots, self.ks, self.vs, validate=False)
        self.q = {b: torch.randn(b, KV_HQ, KV_D, generator=g, device=device).to(torch.bfloat16) for b in KV_BATCH}
        self.perm_gen = torch.Generator().manual_seed(77)
        torch.cuda.synchronize()

    def tables(self, batch: int, ctx: int, max_tables: int = 16):
        torch = self.torch
        per = (ctx + KV_BS - 1) // KV_BS
        count = max(1, min(max_tables, self.num_blocks // (batch * per)))
        perm = torch.randperm(self.num_blocks, generator=self.perm_gen)
        out = []
        for r in range(count):
            ids = perm[r * batch * per:(r + 1) * batch * per].reshape(batch, per)
            out.append(ids.to(torch.int32).to(self.device))
        return out


def kv_attention_bench(kvs: KVSetup, steps: int) -> dict:
    """µs per decode step and per token, and GB/s, of paged decode attention per config."""
    torch = kvs.torch
    op = torch.ops.vllm_ascend_hif8.hif8_paged_decode_attention
    scale = KV_D ** -0.5
    res = {}
    for batch in KV_BATCH:
        for ctx in KV_CTX:
            lens = torch.full((batch,), ctx, dtype=torch.int32, device=kvs.device)
            # Each graph replays KV_CALLS_PER_GRAPH decode steps over different
            # tables (disjoint pages), so launch gaps between replays are
            # amortised as they are between layers of a real decode step.
            tables = kvs.tables(batch, ctx)
            per = min(KV_CALLS_PER_GRAPH, len(tables))
            graphs = []
            for g0 in range(0, len(tables) - per + 1, per):
                def fn(ts=tables[g0:g0 + per]):
                    for table in ts:
                        op(kvs.q[batch], kvs.kc, kvs.vc, table, lens, scale, ctx)
                graphs.append(capture(torch, fn))
            ms = time_graphs(torch, graphs, max(steps // per, 2 * len(graphs))) / per
            nbytes = kv_attention_bytes([ctx] * batch)
            gbs = nbytes / (ms * 1e-3) / 1e9
            res[f"b{batch}_ctx{ctx}"] = {"us_per_step": round(ms * 1e3, 3), "us_per_token": round(ms * 1e3 / batch, 3),
                                         "bytes": nbytes, "GBps": round(gbs, 1),
                                         "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "tables": len(graphs) * per}
            log(f"kv attention b={batch} ctx={ctx}: {ms * 1e3:.2f} us/step, {gbs:.0f} GB/s")
    return res


def kv_write_bench(kvs: KVSetup) -> dict:
    """Fused KV write (quant + pack + scatter) for a decode step (4 tokens) and a 4096-token prefill."""
    torch = kvs.torch
    op = torch.ops.vllm_ascend_hif8.hif8_kv_cache_write
    res = {}
    for tokens in (4, 4096):
        k = torch.randn(tokens, KV_HKV, KV_D, device=kvs.device).to(torch.bfloat16)
        v = torch.randn(tokens, KV_HKV, KV_D, device=kvs.device).to(torch.bfloat16)
        slots = torch.randperm(kvs.num_blocks * KV_BS, device=kvs.device)[:tokens].to(torch.int64)

        def fn():
            for _ in range(10):
                op(k, v, kvs.kc, kvs.vc, slots, kvs.ks, kvs.vs, None)
        ms = time_graphs(torch, [capture(torch, fn)], 3) / 10
        gbs = kv_write_bytes(tokens) / (ms * 1e-3) / 1e9
        res[f"tokens{tokens}"] = {"us": round(ms * 1e3, 3), "bytes": kv_write_bytes(tokens), "GBps": round(gbs, 1),
                                  "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
    return res


def kv_cpu_baseline(budget_s: float = 6.0) -> dict:
    """paged_attention_reference (numpy oracle, reference bf16 roundings) on batch 1, ctx 4096."""
    import numpy as np

    from oracle import hif8_oracle as o

    rng = np.random.default_rng(1)
    ctx, pages = 4096, 4096 // KV_BS
    kc = np.empty((pages, KV_BS, KV_HKV, KV_D + 4), np.uint8)
    vc = np.empty_like(kc)
    for c in (kc, vc):
        data, scale = o.quantize_kv_rows_static(rng.standard_normal((ctx, KV_HKV, KV_D)).astype(np.float32),
                                                np.full(KV_HKV, 4.5 / HIF8_MAX, np.float32))
        c[:] = o.pack_kv_rows(data, scale).reshape(c.shape)
    q = o.round_bf16(rng.standard_normal((1, KV_HQ, KV_D)).astype(np.float32))
    table = rng.permutation(pages)[None, :]
    done, t0 = 0, time.perf_counter()
    while True:
        o.paged_attention_reference(q, kc, vc, table, [ctx], KV_BS, KV_D ** -0.5, rounding="bf16")
        done += 1
        if time.perf_counter() - t0 > budget_s:
            break
    elapsed = time.perf_counter() - t0
    return {"value": round(elapsed / done * 1e6, 1), "unit": "us/token", "cores": 1, "kind": "port",
            "sample": f"{done} decode step(s) of paged_attention_reference (numpy oracle), batch 1, ctx 4096, "
                      f"{elapsed:.1f} s"}


def capture(torch, fn):
    """Capture fn() into a HIP graph after one eager warm-up run on a side stream."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    return graph


def time_graphs(torch, graphs, reps: int) -> float:
    """Average milliseconds per replay of graphs[i % len] (HIP events on the replay stream)."""
    for g in graphs:
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(reps):
        graphs[i % len(graphs)].replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def time_rotated(torch, launch, count: int, per: int = 20, min_launches: int = MIN_TIMED_LAUNCHES):
    """Per-launch time (ms) of launch(i) for i over `count` rotated operand
    copies: graphs of `per` launches covering every copy once per cycle,
    replayed (after one warm-up replay each) until >= min_launches launches
    ran, each replay timed with HIP events on the replay stream.  Returns
    (median, mean) over the replays."""
    graphs = []
    for g0 in range(0, count, per):
        def fn(g0=g0):
            for i in range(per):
                launch((g0 + i) % count)
        graphs.append(capture(torch, fn))
    for g in graphs:
        g.replay()
    torch.cuda.synchronize()
    reps = max(len(graphs), -(-min_launches // per))
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for r, (a, b) in enumerate(ev):
        a.record()
        graphs[r % len(graphs)].replay()
        b.record()
    torch.cuda.synchronize()
    times = sorted(a.elapsed_time(b) / per for a, b in ev)
    return times[len(times) // 2], sum(times) / len(times)


def rotation(st: "Setup", name: str):
    """Weight copies (codes, channel scale) of one projection totalling >= ROTATE_BYTES:
    the Setup's N_COPIES plus clones, made once and kept."""
    if name not in st.rot:
        base = [st.weights[c][name] for c in range(N_COPIES)]
        n, k = base[0][0].shape
        need = max(N_COPIES, -(-ROTATE_BYTES // (n * k)))
        st.rot[name] = base + [(base[i % N_COPIES][0].clone(), base[i % N_COPIES][1]) for i in range(need - N_COPIES)]
    return st.rot[name]


def gemv_plan(m: int, n: int, k: int, kind: int = 0):
    """(kernel name, grid) of the GEMV the library launches for these sizes
    (hif8_gemv_launch_plan; kind 0 = code activations, 2 = bf16 x with a
    fixed scale)."""
    import ctypes

    lib = ctypes.CDLL(str(HOST_LIB))
    f = lib.hif8_gemv_launch_plan
    f.argtypes = [ctypes.c_int64] * 3 + [ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t,
                                         ctypes.POINTER(ctypes.c_int64)]
    buf = ctypes.create_string_buffer(160)
    grid = ctypes.c_int64()
    if f(m, n, k, kind, buf, len(buf), ctypes.byref(grid)) != 0:
        raise RuntimeError("hif8_gemv_launch_plan failed")
    return buf.value.decode(), grid.value


def fused_one_launch(m: int, n: int, k: int) -> bool:
    """Whether soft_static_fused_linear runs one launch for these sizes (the
    torch op's rule, with its knobs HIF8_FUSED_MAX_N / HIF8_FUSED_MAX_K /
    HIF8_FUSED_MULTI_MAX_N): every one-row call (unless the first two cap N
    or K), or several rows with N <= 2048 whose fused-kind plan is the MFMA-4
    GEMV; otherwise static quant + GEMV."""
    if m == 1:
        cap_n, cap_k = os.environ.get("HIF8_FUSED_MAX_N"), os.environ.get("HIF8_FUSED_MAX_K")
        return (not cap_n or n <= int(cap_n)) and (not cap_k or k <= int(cap_k))
    return (n <= int(os.environ.get("HIF8_FUSED_MULTI_MAX_N") or 2048)
            and gemv_plan(m, n, k, 2)[0].startswith("gemv_mfma4_kernel"))


def decode_step_fn(st: Setup, copy: int, fused: bool = False):
    """One decode sweep through the scheme, or through the fused static-quant GEMV."""
    native, torch = st.native, st.torch

    def step():
        for m in DECODE_M:
            for name, n, k in LAYER:
                x, s = st.x[(m, k)]
                if fused:
                    w, ws = st.weights[copy][name]
                    native.soft_static_fused_linear(x, w, s, ws, None, output_dtype=torch.bfloat16)
                else:
                    st.method.apply(st.layers[copy][name], x)
    return step


def per_kernel_table(st: Setup) -> dict:
    """Per-launch time of each GEMV / GEMM / quant: the median over >= 100
    launches (graphs of 20, or 5 above M = 4) rotating >= 768 MB of weight
    copies, so the Infinity Cache cannot serve them.

    GEMV rows name the kernel and grid the library launches (and every
    one-row projection also has a ``_fused`` row: the scheme's default route
    for one token row, the fused static-quant op).  Each fused row carries
    ``quant_then_gemv_us``: the same projection as static quant + GEMV, two
    launches per call."""
    torch, native = st.torch, st.native
    table = {}
    for m in DECODE_M + PREFILL_M:
        for name, n, k in LAYER:
            x, s = st.x[(m, k)]
            q, rs = native.static_quant(x, s)
            rot = rotation(st, name)
            per = 20 if m <= 4 else 5

            def lin(i, q=q, rs=rs, rot=rot):
                native.soft_linear(q, rot[i][0], rs, rot[i][1], None, output_dtype=torch.bfloat16)
            med, mean = time_rotated(torch, lin, len(rot), per)
            entry = {"us": round(med * 1e3, 3), "us_mean": round(mean * 1e3, 3), "copies": len(rot)}
            if m <= 4:
                gbs = gemv_bytes(m, n, k) / (med * 1e-3) / 1e9
                kern, grid = gemv_plan(m, n, k)
                entry.update(kernel="gemv", launch=kern, grid=grid, bytes=gemv_bytes(m, n, k), GBps=round(gbs, 1),
                             frac_hbm=round(gbs / HBM_PEAK_GBS, 4))
            else:
                tf = 2.0 * m * n * k / (med * 1e-3) / 1e12
                entry.update(kernel="gemm", flops=2 * m * n * k, TFLOPs=round(tf, 1),
                             frac_bf16=round(tf / BF16_PEAK_TFLOPS, 4))
            table[f"{name}_m{m}"] = entry
            if m <= 4:
                def fused(i, x=x, s=s, rot=rot):
                    native.soft_static_fused_linear(x, rot[i][0], s, rot[i][1], None, output_dtype=torch.bfloat16)
                med, _ = time_rotated(torch, fused, len(rot), per)

                def two(i, x=x, s=s, rot=rot):  # the same work as two launches (static quant, then the GEMV)
                    qq, rr = native.static_quant(x, s)
                    native.soft_linear(qq, rot[i][0], rr, rot[i][1], None, output_dtype=torch.bfloat16)
                med2, _ = time_rotated(torch, two, len(rot), per)
                fb = gemv_bytes(m, n, k) + m * k  # bf16 x instead of u8 codes
                gbs = fb / (med * 1e-3) / 1e9
                kern, grid = gemv_plan(m, n, k, 2)
                table[f"{name}_m{m}_fused"] = {"kernel": "fused_quant_gemv", "us": round(med * 1e3, 3),
                                               "copies": len(rot), "bytes": fb,
                                               "GBps": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                               "quant_then_gemv_us": round(med2 * 1e3, 3),
                                               "launch": kern if fused_one_launch(m, n, k)
                                               else "hif8_static_quant + code GEMV", "grid": grid}
    for m, k in ((4096, 4096), (4096, 12288), (512, 4096), (1, 4096), (4, 12288)):
        x, s = st.x[(m, k)]
        xs = [x] + [x.clone() for _ in range(-(-ROTATE_BYTES // (2 * m * k)) - 1)] if m > 4 else [x]
        med, _ = time_rotated(torch, lambda i, xs=xs, s=s: native.static_quant(xs[i], s), len(xs), 10)
        del xs
        gbs = quant_bytes(m, k) / (med * 1e-3) / 1e9
        table[f"static_quant_m{m}_k{k}"] = {"kernel": "static_quant", "us": round(med * 1e3, 3),
                                            "bytes": quant_bytes(m, k), "GBps": round(gbs, 1),
                                            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
    return table


def decoded_weight_gemm(st: Setup) -> dict:
    """Prefill GEMMs with the weight kept decoded to bf16 (the opt-in
    HIF8_PREFILL_BF16_WEIGHTS=1 route, soft_hif8_gemm_decoded_weight): per
    shape and per layer at M in PREFILL_M, median over >= 100 launches in
    graphs of 5 rotating >= 768 MB of decoded copies.  The one-time decodes
    are made before timing (they happen once per model load)."""
    torch, native = st.torch, st.native
    res = {}
    for name, n, k in LAYER:
        rot = rotation(st, name)
        decoded = [native.decode_weight(rot[i][0]) for i in range(-(-ROTATE_BYTES // (2 * n * k)))]
        for m in PREFILL_M:
            x, s = st.x[(m, k)]
            q, rs = native.static_quant(x, s)

            def fn(i, q=q, rs=rs, rot=rot, decoded=decoded):
                native.soft_linear_decoded_weight(q, decoded[i], rs, rot[i][1], None, output_dtype=torch.bfloat16)
            med, _ = time_rotated(torch, fn, len(decoded), 5)
            tf = 2.0 * m * n * k / (med * 1e-3) / 1e12
            res[f"{name}_m{m}"] = {"us": round(med * 1e3, 3), "TFLOPs": round(tf, 1),
                                   "frac_bf16": round(tf / BF16_PEAK_TFLOPS, 4), "copies": len(decoded)}
        del decoded
        torch.cuda.empty_cache()
    for m in PREFILL_M:
        fl_total = sum(2.0 * m * n * k for _, n, k in LAYER)
        us_total = sum(res[f"{name}_m{m}"]["us"] for name, _, _ in LAYER)
        tf = fl_total / (us_total * 1e-6) / 1e12
        res[f"layer_m{m}"] = {"TFLOPs": round(tf, 1), "frac_bf16": round(tf / BF16_PEAK_TFLOPS, 4),
                              "us_per_layer": round(us_total, 1)}
    return res


def aux_kernels(torch, native, device) -> dict:
    """The decode ops beside the fused path: hif8_scaled_decode of KV rows
    (16384 rows x 256 codes -> bf16), the embedding gather-decode (vocab
    151936 x 4096 table; 4 decode tokens and a 512-token prompt) and the
    legacy dynamic quant (M in {1, 4096}, K 4096).  Bytes: codes + scales
    read, bf16 written (+ ids); dynamic quant: bf16 in, codes + scales out."""
    res = {}
    g = torch.Generator(device=device).manual_seed(5)
    rows, k = 16384, 256
    data = torch.randint(0, 111, (rows, k), generator=g, device=device, dtype=torch.uint8)
    scale = torch.rand(rows, generator=g, device=device)

    def dec():
        for _ in range(10):
            native.scaled_decode(data, scale)
    ms = time_graphs(torch, [capture(torch, dec)], 3) / 10
    nbytes = rows * k * 3 + rows * 4
    res["scaled_decode_16384x256"] = {"us": round(ms * 1e3, 3), "bytes": nbytes,
                                      "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    vocab, dim = 151936, 4096
    table = torch.randint(0, 111, (vocab, dim), generator=g, device=device, dtype=torch.uint8)
    tscale = torch.rand(vocab, generator=g, device=device)
    for tokens in (4, 512):
        ids = torch.randint(0, vocab, (tokens,), generator=g, device=device)

        def emb(ids=ids):
            for _ in range(10):
                native.embedding_lookup(table, tscale, ids, validate=False)
        ms = time_graphs(torch, [capture(torch, emb)], 3) / 10
        nbytes = tokens * (dim * 3 + 4 + 8)
        res[f"embedding_{tokens}tok_x{dim}"] = {"us": round(ms * 1e3, 3), "bytes": nbytes,
                                                "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    del table
    # The legacy dynamic-scale path: per-row amax + encode (bf16 in, codes and
    # row scales out; the row is read twice, the second time from cache).
    for m, kk in ((1, 4096), (4096, 4096)):
        x = torch.randn(m, kk, generator=g, device=device).to(torch.bfloat16)

        def dq(x=x):
            for _ in range(10):
                native.dynamic_quant(x)
        ms = time_graphs(torch, [capture(torch, dq)], 3) / 10
        nbytes = m * kk * 3 + m * 4
        res[f"dynamic_quant_m{m}_k{kk}"] = {"us": round(ms * 1e3, 3), "bytes": nbytes,
                                            "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    return res


def measured_ceilings(torch, device) -> dict:
    """Context for the rooflines: a plain device copy (HBM read + write) and
    torch's bf16 matmul (hipBLASLt) on the prefill shapes with bf16 operands,
    i.e. the same GEMMs without any HiF8 decode."""
    src = torch.empty(512 * 2 ** 20, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)

    def cp():
        for _ in range(5):
            dst.copy_(src)
    ms = time_graphs(torch, [capture(torch, cp)], 3) / 5
    copy_gbs = 2 * src.numel() / (ms * 1e-3) / 1e9
    del src, dst
    gemm = {}
    for m in PREFILL_M:
        for name, n, k in LAYER:
            a = torch.randn(m, k, device=device).to(torch.bfloat16)
            w = torch.randn(n, k, device=device).to(torch.bfloat16)

            def mm(a=a, w=w):
                for _ in range(3):
                    torch.matmul(a, w.t())
            ms = time_graphs(torch, [capture(torch, mm)], 5) / 3
            tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
            gemm[f"{name}_m{m}"] = {"us": round(ms * 1e3, 2), "TFLOPs": round(tf, 1),
                                    "frac_bf16": round(tf / BF16_PEAK_TFLOPS, 4)}
    return {"hbm_copy_GBps": round(copy_gbs, 1), "hbm_copy_frac": round(copy_gbs / HBM_PEAK_GBS, 4),
            "hipblaslt_bf16_gemm": gemm}


def cpu_baseline(budget_s: float = 5.0) -> dict:
    """The numpy oracle's decode-GEMV sweep on the host (single-threaded numpy gather + BLAS)."""
    import numpy as np

    from oracle import hif8_oracle as o

    rng = np.random.default_rng(0)
    step_bytes = sum(quant_bytes(m, k) + gemv_bytes(m, n, k) for m in DECODE_M for _, n, k in LAYER)
    weights = {}
    for name, n, k in LAYER:
        weights[name] = (rng.integers(0, 111, (n, k), dtype=np.uint8), (rng.random(n, dtype=np.float32) + 0.5) * 1e-5)
    xs = {(m, k): rng.standard_normal((m, k)).astype(np.float32) for m in DECODE_M for k in (4096, 12288)}
    done, t0 = 0, time.perf_counter()
    while True:
        for m in DECODE_M:
            for name, n, k in LAYER:
                x = xs[(m, k)]
                s = np.array([np.abs(x).max() / HIF8_MAX], np.float32)
                xq, _ = o.static_quant_rows(x, s)
                w, ws = weights[name]
                wd = o.DECODE_F32[w] * ws[:, None]          # decode-LUT weights x channel scale
                _ = (o.DECODE_F32[xq] * s[0]) @ wd.T          # fp32 matmul
        done += 1
        if time.perf_counter() - t0 > budget_s:
            break
    elapsed = time.perf_counter() - t0
    return {"value": round(step_bytes * done / elapsed / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{done} full decode sweep step(s) (M in {{1,4}} x 5 projections, quant + LUT-decode + fp32 "
                      f"matmul) of the numpy oracle, {elapsed:.1f} s, OMP/BLAS threads 1"}


C1_SEED = 20261201
C1_N, C1_K = 12288, 4096


def c1_operands():
    """BASELINE configs[0] on the CPU: x bf16 [1, 4096] ~ N(0, 1) with input_scale =
    absmax / 32768; W fp32 [12288, 4096] ~ N(0, 0.02) with per-row scale = row
    absmax / 32768, encoded by the torch-CPU port of the reference codec (bit-equal
    to the oracle).  One seeded generator drives both, as in tests/_data.py."""
    import torch

    from oracle import torch_cpu

    g = torch.Generator().manual_seed(C1_SEED)
    x = torch.randn(1, C1_K, generator=g, dtype=torch.float32).to(torch.bfloat16)
    s = torch.tensor([float(x.float().abs().max()) / HIF8_MAX], dtype=torch.float32)
    w = torch.randn(C1_N, C1_K, generator=g, dtype=torch.float32) * 0.02
    ws = (w.abs().amax(dim=1) / HIF8_MAX).to(torch.float32)
    wq = torch_cpu.static_quant(w, ws.reshape(-1, 1))
    return x, s, wq, ws


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def c1_cpu_baseline(threads: int, runs: int = 5, warmup: int = 2) -> dict:
    """BASELINE configs[0] timed on the host's CPU threads: the torch-CPU
    restatement of the reference's CPU path - static encode of x (x / scale,
    saturate, LUT encode), then decode-LUT weights x channel scale and one fp32
    matmul with the decoded activation (tests/test_npu_ops.py:334-336).  Median
    of `runs` runs after `warmup`, at `threads` torch threads and at one."""
    import torch

    from oracle import torch_cpu

    x, s, wq, ws = c1_operands()
    nbytes = gemv_bytes(1, C1_N, C1_K) + quant_bytes(1, C1_K)
    out = {}
    for n in (threads, 1):
        torch.set_num_threads(n)
        times = []
        for i in range(warmup + runs):
            t0 = time.perf_counter()
            xq = torch_cpu.static_quant(x.float(), float(s[0]))
            torch_cpu.soft_gemv(xq, s, wq, ws)
            if i >= warmup:
                times.append(time.perf_counter() - t0)
        times.sort()
        med = times[len(times) // 2]
        out[n] = {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "us_per_gemv": round(med * 1e6, 1),
                  "cores": n}
    torch.set_num_threads(threads)
    return out


def c1_gpu(torch, native, device) -> dict:
    """BASELINE configs[0] on the GPU: static_quant + soft_linear (M = 1, N 12288,
    K 4096 -> the GEMV kernel) on the seeded weights, 6 weight copies (302 MB)
    rotated past the Infinity Cache; graphs of 20 launches."""
    x, s, wq, ws = c1_operands()
    wd = wq.to(device)
    copies = [(wd if i == 0 else wd.clone(), ws.to(device)) for i in range(-(-ROTATE_BYTES // wq.numel()))]
    xd, sd = x.to(device), s.to(device)
    q, rs = native.static_quant(xd, sd)

    def both(i):
        qq, rr = native.static_quant(xd, sd)
        native.soft_linear(qq, copies[i][0], rr, copies[i][1], None, output_dtype=torch.bfloat16)

    def gemv(i):
        native.soft_linear(q, copies[i][0], rs, copies[i][1], None, output_dtype=torch.bfloat16)

    def fused(i):
        native.soft_static_fused_linear(xd, copies[i][0], sd, copies[i][1], None, output_dtype=torch.bfloat16)
    ms_both, _ = time_rotated(torch, both, len(copies))
    ms_gemv, _ = time_rotated(torch, gemv, len(copies))
    ms_fused, _ = time_rotated(torch, fused, len(copies))
    kern, grid = gemv_plan(1, C1_N, C1_K)
    gb = gemv_bytes(1, C1_N, C1_K)
    qb = quant_bytes(1, C1_K)
    res = {"workload": "BASELINE configs[0]: M=1 GEMV, N 12288, K 4096, seeded fp32 N(0,0.02) weights encoded "
                       "with per-row absmax/32768 scales, x ~ N(0,1) bf16 with a static absmax/32768 scale",
           "gemv_launch": kern, "gemv_grid": grid, "weight_copies": len(copies),
           "gemv_us": round(ms_gemv * 1e3, 3), "gemv_bytes": gb,
           "gemv_GBps": round(gb / (ms_gemv * 1e-3) / 1e9, 1),
           "gemv_frac_hbm": round(gb / (ms_gemv * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "quant_plus_gemv_us": round(ms_both * 1e3, 3),
           "quant_plus_gemv_GBps": round((gb + qb) / (ms_both * 1e-3) / 1e9, 1),
           "scheme_route_us": round(ms_fused * 1e3, 3),
           "scheme_route": "the scheme's default for one token row: the fused static-quant op, "
                           + ("one launch of " + gemv_plan(1, C1_N, C1_K, 2)[0] if fused_one_launch(1, C1_N, C1_K)
                              else "static quant + the code GEMV inside it")}
    del copies
    return res


def prefill_attention_flops(ctx: int, q_len: int) -> int:
    """QK^T and PV multiply-adds of one request's causal rows (row i sees ctx - q_len + i + 1 keys)."""
    visible = sum(ctx - q_len + i + 1 for i in range(q_len))
    return 4 * KV_HQ * KV_D * visible


def prefill_attention_bench(kvs: "KVSetup") -> dict:
    """Multi-token paged attention (hif8_paged_prefill_attention) over the same
    HiF8 page pool: a whole 512-token prompt, 512- and 17-token chunks at the
    end of a 4096-token context, batch 1 and 4; graphs of 4 calls over
    disjoint random pages.  Work = causal QK^T + PV flops."""
    torch = kvs.torch
    res = {}
    g = torch.Generator(device=kvs.device).manual_seed(6)
    for batch, ctx, q_len in ((1, 512, 512), (1, 4096, 512), (4, 4096, 512), (1, 4096, 17), (4, 4096, 17)):
        tables = kvs.tables(batch, ctx, max_tables=4)
        q = torch.randn(batch * q_len, KV_HQ, KV_D, generator=g, device=kvs.device).to(torch.bfloat16)
        lens = torch.full((batch,), ctx, dtype=torch.int32, device=kvs.device)
        loc = torch.arange(0, batch * q_len + 1, q_len, dtype=torch.int32, device=kvs.device)
        op = torch.ops.vllm_ascend_hif8.hif8_paged_prefill_attention

        def fn(tables=tables, q=q, lens=lens, loc=loc):
            for t in tables:
                op(q, kvs.kc, kvs.vc, t, loc, lens, KV_D ** -0.5, q_len, ctx, True)
        ms = time_graphs(torch, [capture(torch, fn)], 5) / len(tables)
        fl = batch * prefill_attention_flops(ctx, q_len)
        tf = fl / (ms * 1e-3) / 1e12
        res[f"b{batch}_ctx{ctx}_q{q_len}"] = {"us": round(ms * 1e3, 2), "flops": fl, "TFLOPs": round(tf, 1),
                                              "frac_bf16": round(tf / BF16_PEAK_TFLOPS, 4)}
        log(f"prefill attention b={batch} ctx={ctx} q={q_len}: {ms * 1e3:.1f} us, {tf:.1f} TFLOP/s")
    return res


def profile_pass(st: Setup, reps: int = 3) -> None:
    """Eager launches for counter collection (rocprofv3 --pmc ...).

    Known-size calibration kernels first: a torch copy of 64 MiB (read + write)
    and an fp32 sum over the same 64 MiB (a plain streaming read with 16-byte
    vector loads, the load width of the GEMV).  Then every decode GEMV, static
    quant and prefill GEMM launch `reps` times, and the fused op per decode
    (M, shape) `reps` times."""
    torch, native = st.torch, st.native
    src = torch.empty(64 << 20, dtype=torch.uint8, device=st.device).fill_(3)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        src.view(torch.float32).sum()
    torch.cuda.synchronize()
    for m in DECODE_M + PREFILL_M:
        for name, n, k in LAYER:
            x, s = st.x[(m, k)]
            for i in range(reps):
                q, rs = native.static_quant(x, s)
                w, ws = st.weights[i % N_COPIES][name]
                native.soft_linear(q, w, rs, ws, None, output_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    # The fused op (the scheme's default for decode-sized inputs), `reps` times per (M, shape).
    for m in DECODE_M:
        for name, n, k in LAYER:
            x, s = st.x[(m, k)]
            for i in range(reps):
                w, ws = st.weights[i % N_COPIES][name]
                native.soft_static_fused_linear(x, w, s, ws, None, output_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    log("profile pass: linear done")
    # KV path: decode attention (b4 ctx16384, b1 ctx512), the fused cache write
    # of 4096 tokens, multi-token attention (b1, 512 rows over 4096 tokens);
    # each `reps` times over distinct random pages.
    kvs = KVSetup(torch, st.device)
    for batch, ctx in ((4, 16384), (1, 512)):
        lens = torch.full((batch,), ctx, dtype=torch.int32, device=st.device)
        for t in kvs.tables(batch, ctx, max_tables=reps):
            torch.ops.vllm_ascend_hif8.hif8_paged_decode_attention(kvs.q[batch], kvs.kc, kvs.vc, t, lens,
                                                                   KV_D ** -0.5, ctx)
    torch.cuda.synchronize()
    g = torch.Generator(device=st.device).manual_seed(3)
    k = torch.randn(4096, KV_HKV, KV_D, generator=g, device=st.device).to(torch.bfloat16)
    v = torch.randn(4096, KV_HKV, KV_D, generator=g, device=st.device).to(torch.bfloat16)
    perm = torch.randperm(kvs.num_blocks * KV_BS, generator=kvs.perm_gen)[:4096].to(st.device)
    for _ in range(reps):
        torch.ops.vllm_ascend_hif8.hif8_kv_cache_write(k, v, kvs.kc, kvs.vc, perm, kvs.ks, kvs.vs, None)
    q = torch.randn(512, KV_HQ, KV_D, generator=g, device=st.device).to(torch.bfloat16)
    loc = torch.tensor([0, 512], dtype=torch.int32, device=st.device)
    lens = torch.tensor([4096], dtype=torch.int32, device=st.device)
    for t in kvs.tables(1, 4096, max_tables=reps):
        torch.ops.vllm_ascend_hif8.hif8_paged_prefill_attention(q, kvs.kc, kvs.vc, t, loc, lens, KV_D ** -0.5,
                                                                512, 4096, True)
    torch.cuda.synchronize()
    log("profile pass done")


def committed_traffic(row: str, kernel: str, grid: int):
    """HBM bytes per launch of `row` measured with rocprofv3 --pmc
    (profiles/pmc_traffic.json) and a note; None unless the profile was taken
    on the same kernel (name with template arguments) and grid as the launch
    timed here."""
    path = REPO / "profiles" / "pmc_traffic.json"
    if not path.exists():
        return None, "no committed PMC profile"
    entry = json.loads(path.read_text()).get("kernels", {}).get(row)
    if entry is None:
        return None, f"no PMC entry for {row}"
    if entry.get("kernel") != kernel or int(entry.get("grid", -1)) != int(grid):
        log(f"PMC profile of {row} is for {entry.get('kernel')} x {entry.get('grid')}, the bench times {kernel} x {grid}")
        return None, (f"refused: the committed profile measured {entry.get('kernel')} x {entry.get('grid')} "
                      f"workgroups, the bench times {kernel} x {grid}")
    return entry.get("traffic_bytes"), (f"profiles/pmc_traffic.json: FETCH_SIZE x {json.loads(path.read_text())['fetch_scale']:.3f} "
                                        f"+ WRITE_SIZE of {kernel} x {grid}")


def _median_time(fn, threads: int, runs: int, warmup: int) -> float:
    import torch

    torch.set_num_threads(threads)
    times = []
    for i in range(warmup + runs):
        t0 = time.perf_counter()
        fn()
        if i >= warmup:
            times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2]


def gemm_cpu_baseline(threads: int, runs: int = 5, warmup: int = 2) -> dict:
    """BASELINE configs[2] on the host, the q projection at M = 512 (512 x 4096
    x 4096): the torch-CPU port of the reference's CPU path - static encode of
    x, then decode-LUT weights x channel scale and one fp32 matmul with the
    decoded activation (tests/test_npu_ops.py:334-336).  Median of `runs`
    after `warmup`, at `threads` torch threads and at one."""
    import torch

    from oracle import torch_cpu

    m, n, k = 512, 4096, 4096
    g = torch.Generator().manual_seed(C1_SEED + 2)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    s = torch.tensor([float(x.float().abs().max()) / HIF8_MAX], dtype=torch.float32)
    w = torch.randn(n, k, generator=g) * 0.02
    ws = (w.abs().amax(dim=1) / HIF8_MAX).to(torch.float32)
    wq = torch_cpu.static_quant(w, ws.reshape(-1, 1))

    def run():
        xq = torch_cpu.static_quant(x.float(), float(s[0]))
        torch_cpu.soft_gemv(xq, s.expand(m), wq, ws)
    out = {}
    for t in (threads, 1):
        med = _median_time(run, t, runs, warmup)
        out[t] = {"value": round(2.0 * m * n * k / med / 1e12, 4), "unit": "TFLOP/s", "ms_per_gemm": round(med * 1e3, 2),
                  "cores": t}
    torch.set_num_threads(threads)
    return {"value": out[threads]["value"], "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"BASELINE configs[2] q projection at M=512 (512x4096x4096, 17.2 GFLOP): torch-CPU port of the "
                      f"reference CPU path (static encode of x, decode-LUT weights x scale, fp32 matmul), median of "
                      f"{runs} after {warmup} warm-up runs, {out[threads]['ms_per_gemm']} ms per GEMM at {threads} "
                      f"threads", "nproc": os.cpu_count(), "cpu_model": cpu_model(), "single_thread": out[1]}


def kv_cpu_baseline_torch(threads: int, runs: int = 5, warmup: int = 2) -> dict:
    """BASELINE configs[3] at batch 4, ctx 4096 on the host: the torch-CPU port
    of the reference's paged_attention_reference (kv_cache.py:314-372; gather,
    decode x row scale to bf16, GQA repeat, bf16 einsums, fp32 softmax) over a
    HiF8 cache written by the numpy oracle.  Median of `runs` after `warmup`
    at `threads` torch threads and at one; us per token = step time / 4."""
    import numpy as np
    import torch

    from oracle import hif8_oracle as o
    from oracle import torch_cpu

    batch, ctx = 4, 4096
    pages = batch * ctx // KV_BS
    rng = np.random.default_rng(2)
    kc = np.zeros((pages, KV_BS, KV_HKV, KV_D + 4), np.uint8)
    vc = np.zeros_like(kc)
    for c in (kc, vc):
        vals = rng.standard_normal((pages * KV_BS, KV_HKV, KV_D)).astype(np.float32)
        data, sc = o.quantize_kv_rows_static(vals, (np.abs(vals).max(axis=(0, 2)) / HIF8_MAX).astype(np.float32))
        o.scatter_kv_rows(c, o.pack_kv_rows(data, sc), np.arange(pages * KV_BS), KV_BS)
    table = torch.from_numpy(rng.permutation(pages).reshape(batch, ctx // KV_BS))
    q = torch.randn(batch, KV_HQ, KV_D, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    kct, vct = torch.from_numpy(kc), torch.from_numpy(vc)

    def run():
        torch_cpu.paged_decode_attention(q, kct, vct, table, [ctx] * batch, KV_D ** -0.5)
    out = {}
    for t in (threads, 1):
        med = _median_time(run, t, runs, warmup)
        out[t] = {"value": round(med * 1e6 / batch, 1), "unit": "us/token", "ms_per_step": round(med * 1e3, 2),
                  "cores": t}
    torch.set_num_threads(threads)
    return {"value": out[threads]["value"], "unit": "us/token", "cores": threads, "kind": "port",
            "sample": f"BASELINE configs[3] batch 4, ctx 4096 (Hq 16, Hkv 4, D 256, 128-token pages): torch-CPU port of "
                      f"the reference's paged_attention_reference, one decode step, median of {runs} after {warmup} "
                      f"warm-up runs, {out[threads]['ms_per_step']} ms per step at {threads} threads",
            "nproc": os.cpu_count(), "cpu_model": cpu_model(), "single_thread": out[1]}


E2E_PROMPT, E2E_NEW = 512, 256


def e2e_decode(torch, device) -> dict:
    """greedy decode through the static scheme of a
    random-init Qwen3.5-9B-shaped hybrid (hif8_rocm.synthetic_model), random
    prompt ids, 512 prompt + 256 new tokens at batch 1 and 4.  Output tok/s
    = batch x 256 / (prefill + 255 decode steps at the graph-replay rate);
    the first decode step and the graph recording (done once per process by a
    server) are reported apart."""
    from hif8_rocm.synthetic_model import HybridConfig, HybridModel, generate

    cfg = HybridConfig()
    t0 = time.perf_counter()
    model = HybridModel(cfg, device, seed=0)
    model.calibrate(batch=1, tokens=128)
    torch.cuda.synchronize()
    res = {"workload": "BASELINE configs[4]: random-init Qwen3.5-9B-shaped hybrid (32 layers, hidden 4096, "
                       "full attention every 4th layer with HiF8 KV, gated-delta-rule layers, intermediate "
                       "12288, vocab 151936); every projection W8A8 HiF8 static through the scheme, embedding "
                       "HiF8 SOFT, norms / conv / recurrence in bf16-fp32 glue kernels, bf16 LM head (library bf16 GEMV up "
                       "to 4 rows); greedy, random ids",
           "prompt_tokens": E2E_PROMPT, "new_tokens": E2E_NEW, "build_and_calibrate_s": round(time.perf_counter() - t0, 2)}
    g = torch.Generator(device=device).manual_seed(9)
    # b1_single_row_fusion: batch 1 again with the glue-kernel input quant
    # off, so every one-row projection (qkv / qkvz, gate_up, o / out, down)
    # goes through the scheme's fused static-quant op (HIF8_STATIC_FUSED_SINGLE_ROW,
    # the default), one launch for K <= 4096 and N < 16384 (same tokens).
    for b, key, single in ((1, "b1", False), (4, "b4", False), (1, "b1_single_row_fusion", True)):
        prompt = torch.randint(0, cfg.vocab, (b, E2E_PROMPT), generator=g, device=device)
        if single:
            os.environ["HIF8_STATIC_FUSED_SINGLE_ROW"] = "1"
            model.fuse_input_quant = False
        try:
            generate(model, prompt[:, :64], 4)  # warm-up: allocator, kernels, graph capture path
            _, tm = generate(model, prompt, E2E_NEW)
        finally:
            os.environ.pop("HIF8_STATIC_FUSED_SINGLE_ROW", None)
            model.fuse_input_quant = True
        step_s = tm["decode"] / tm["decode_steps"]
        total = tm["prefill"] + step_s * (E2E_NEW - 1)
        res[key] = {"prefill_ms": round(tm["prefill"] * 1e3, 2), "ms_per_decode_step": round(step_s * 1e3, 3),
                    "first_step_and_graph_record_ms": round(tm["setup"] * 1e3, 1),
                    "decode_tok_per_s": round(b / step_s, 1),
                    "output_tok_per_s": round(b * E2E_NEW / total, 1)}
        log(f"e2e {key}: prefill {tm['prefill'] * 1e3:.1f} ms, {step_s * 1e3:.3f} ms/step, "
            f"{res[key]['output_tok_per_s']} output tok/s")
    del model
    torch.cuda.empty_cache()
    return res


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-e2e", action="store_true", help="skip the synthetic end-to-end decode (config 5)")
    ap.add_argument("--profile-pass", action="store_true",
                    help="eager launches only, for rocprofv3 counter collection; prints no JSON")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

    cpu = kv_cpu = gemm_cpu = None
    # The host's thread share: OMP_NUM_THREADS where the pool sets it (16 per GPU
    # on the GPU boxes), else every CPU; never more than the CPUs present.
    nproc = os.cpu_count() or 1
    threads = min(int(os.environ.get("OMP_NUM_THREADS") or nproc), nproc)
    if not args.no_cpu_baseline and not args.profile_pass:
        for var in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS"):
            os.environ[var] = "1"
        log("cpu baseline (numpy oracle decode sweep, 1 thread) ...")
        sweep_cpu = cpu_baseline()
        log(f"cpu baseline sweep {sweep_cpu['value']} GB/s")
        kv_cpu = kv_cpu_baseline()
        log(f"kv cpu baseline {kv_cpu['value']} us/token")
        log(f"cpu baseline C1 (torch-CPU port, {threads} and 1 threads) ...")
        c1 = c1_cpu_baseline(threads)
        model = cpu_model()
        cpu = {"value": c1[threads]["value"], "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"BASELINE configs[0] (M=1 GEMV 12288x4096 + static quant of x): torch-CPU port of the "
                         f"reference CPU path (codec encode, decode-LUT weights x scale, fp32 matmul), median of 5 "
                         f"after 2 warm-up runs, {c1[threads]['us_per_gemv']} us per GEMV at {threads} threads",
               "nproc": nproc, "cpu_model": model, "single_thread": c1[1], "decode_sweep_numpy_1thread": sweep_cpu}
        log(f"cpu baseline C1: {c1[threads]['value']} GB/s at {threads} threads, {c1[1]['value']} GB/s at 1")
        gemm_cpu = gemm_cpu_baseline(threads)
        log(f"cpu baseline GEMM q M=512: {gemm_cpu['value']} TFLOP/s at {threads} threads, "
            f"{gemm_cpu['single_thread']['value']} at 1")
        kv_cpu_t = kv_cpu_baseline_torch(threads)
        log(f"cpu baseline KV b4 ctx4096: {kv_cpu_t['value']} us/token at {threads} threads, "
            f"{kv_cpu_t['single_thread']['value']} at 1")
        kv_cpu_t["numpy_oracle_1thread_b1_ctx4096"] = kv_cpu
        kv_cpu = kv_cpu_t

    import torch

    from hif8_rocm import native

    native.load_extension()
    device = torch.device("cuda:0")
    log("generating synthetic weights ...")
    st = Setup(torch, native, device)
    if args.profile_pass:
        profile_pass(st)
        return

    log("capturing decode-sweep graphs ...")
    graphs = [capture(torch, decode_step_fn(st, c)) for c in range(N_COPIES)]
    # Untimed settle before the W warm-up steps: ~50 ms of replays, so the
    # shader clock and the caches are in their steady state whatever W the
    # caller passes (a 20-step timed region is only ~2.5 ms of GPU work).
    for i in range(max(0, SETTLE_STEPS - args.warmup)):
        graphs[i % N_COPIES].replay()
    for i in range(args.warmup):
        graphs[i % N_COPIES].replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for i in range(args.steps):
        graphs[i % N_COPIES].replay()
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    gpu_ms = e0.elapsed_time(e1) / args.steps
    step_bytes = sum(quant_bytes(m, k) + gemv_bytes(m, n, k) for m in DECODE_M for _, n, k in LAYER)
    value = step_bytes / (wall_ms * 1e-3) / 1e9
    log(f"decode sweep: {wall_ms * 1e3:.1f} us/step wall, {gpu_ms * 1e3:.1f} us/step events, {value:.1f} GB/s")

    fused = [capture(torch, decode_step_fn(st, c, fused=True)) for c in range(N_COPIES)]
    fused_ms = time_graphs(torch, fused, args.steps)
    fused_gbs = step_bytes / (fused_ms * 1e-3) / 1e9
    log(f"fused single-launch sweep: {fused_ms * 1e3:.1f} us/step, {fused_gbs:.1f} GB/s")

    # The scheme with the reference's routing (HIF8_STATIC_FUSED_SINGLE_ROW=0:
    # every projection as static quant + GEMV; equal outputs).  apply() routes
    # at capture time.
    os.environ["HIF8_STATIC_FUSED_SINGLE_ROW"] = "0"
    two = [capture(torch, decode_step_fn(st, c)) for c in range(N_COPIES)]
    del os.environ["HIF8_STATIC_FUSED_SINGLE_ROW"]
    two_ms = time_graphs(torch, two, args.steps)
    two_gbs = step_bytes / (two_ms * 1e-3) / 1e9
    del two
    log(f"sweep with two-stage one-row projections: {two_ms * 1e3:.1f} us/step, {two_gbs:.1f} GB/s")

    log("per-kernel table ...")
    table = per_kernel_table(st)
    log("prefill GEMMs over decoded weights ...")
    gemm_decoded = decoded_weight_gemm(st)
    log(f"decoded-weight layer: m512 {gemm_decoded['layer_m512']['us_per_layer']} us, "
        f"m4096 {gemm_decoded['layer_m4096']['us_per_layer']} us")
    gemv = [v for v in table.values() if v["kernel"] == "gemv"]
    # The launches of the headline step: every projection through the fused
    # op (one launch where fused_one_launch says so, else static quant + the
    # code GEMV inside the op).  The dominant launch is the longest of them.
    step_rows = [(f"{name}_m{m}_fused" if fused_one_launch(m, n, k) else f"{name}_m{m}")
                 for m in DECODE_M for name, n, k in LAYER]
    dom_key = max(step_rows, key=lambda r: table[r]["us"])
    best_key = max(step_rows, key=lambda r: table[r]["frac_hbm"])
    dom, best = table[dom_key], table[best_key]
    traffic, traffic_note = committed_traffic(dom_key, dom["launch"], dom["grid"])
    gemm_layer = {}
    for m in PREFILL_M:
        fl = sum(table[f"{n}_m{m}"]["flops"] for n, _, _ in LAYER)
        us = sum(table[f"{n}_m{m}"]["us"] for n, _, _ in LAYER)
        tf = fl / (us * 1e-6) / 1e12
        gemm_layer[f"m{m}"] = {"TFLOPs": round(tf, 1), "frac_bf16": round(tf / BF16_PEAK_TFLOPS, 4),
                               "us_per_layer": round(us, 1)}
    gdom = table["gate_up_m4096"]
    gemm_layer["cpu_baseline"] = gemm_cpu
    gemm_layer["roofline"] = {"kernel": "the GEMM call for gate_up 4096x24576x4096 (activation and weight decodes + "
                                        "gemm_dma_kernel<256,256>)",
                              "bound": "mfma", "achieved": gdom["TFLOPs"], "peak": BF16_PEAK_TFLOPS,
                              "unit": "TFLOP/s", "frac": gdom["frac_bf16"], "flops_per_launch": gdom["flops"],
                              "us_per_launch": gdom["us"]}
    all_gemv_gbs = sum(v["bytes"] for v in gemv) / (sum(v["us"] for v in gemv) * 1e-6) / 1e9

    log("configs[0] GEMV ...")
    c1 = c1_gpu(torch, native, device)
    log(f"c1 gemv: {c1['gemv_us']} us, {c1['gemv_GBps']} GB/s")
    log("ceilings (plain copy, hipBLASLt bf16 GEMM) ...")
    ceilings = measured_ceilings(torch, device)
    log("scaled decode and embedding ...")
    aux = aux_kernels(torch, native, device)

    log("KV page pool ...")
    kvs = KVSetup(torch, device)
    kv_attn = kv_attention_bench(kvs, args.steps)
    kv_write = kv_write_bench(kvs)
    log("multi-token (prefill) attention ...")
    prefill_attn = prefill_attention_bench(kvs)
    kv_dom = kv_attn[f"b{KV_BATCH[-1]}_ctx{KV_CTX[-1]}"]
    e2e = None
    if not args.no_e2e:
        del kvs
        log("end-to-end synthetic decode ...")
        e2e = e2e_decode(torch, device)

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "decode GEMV sweep (BASELINE configs[1]): static W8A8 scheme apply = static_quant + "
                        "soft_hif8_gemm, M in {1,4} x q/kv/o/gate_up/down of one 9B-class layer, 5 rotated "
                        "weight copies, HIP-graph replay",
            "operands": "HiF8 u8 weights/activations, bf16 dot products, fp32 accumulate, bf16 out",
            "shapes_nk": [[n, k] for _, n, k in LAYER],
            "m": list(DECODE_M),
            "step_bytes": step_bytes,
        },
        "roofline": {
            "kernel": f"{dom['launch']} x {dom['grid']} workgroups ({dom_key}: the longest launch of the step)",
            "bound": "hbm",
            "achieved": dom["GBps"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_note,
            "bytes_per_launch": dom["bytes"],
            "us_per_launch": dom["us"],
            "timing": f"median over >= {MIN_TIMED_LAUNCHES} launches, graphs of 20 rotating {dom.get('copies')} "
                      f"weight copies, HIP events on the replay stream",
            "best_launch": {"row": best_key, "kernel": f"{best['launch']} x {best['grid']}", "GBps": best["GBps"],
                            "frac": best["frac_hbm"], "us": best["us"]},
        },
        "cpu_baseline": cpu,
        "kv_decode_attention": {
            "workload": "BASELINE configs[3]: paged decode attention, Hq 16, Hkv 4, D 256, page 128, one query "
                        "token per request, per-head static K/V scales, random disjoint pages from a 1.1 GB pool "
                        "rotated per step; bytes = K+V rows (codes + sidecar) + q + out + block-table entries",
            "configs": kv_attn,
            "roofline": {"kernel": "paged_decode_attention_kernel + combine (batch 4, ctx 16384)", "bound": "hbm",
                         "achieved": kv_dom["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": kv_dom["frac_hbm"], "us_per_token": kv_dom["us_per_token"]},
            "cpu_baseline": kv_cpu,
            "kv_cache_write": kv_write,
        },
        "prefill_attention": {
            "workload": "multi-token paged attention over the same HiF8 pages (Hq 16, Hkv 4, D 256, page 128): "
                        "q_len new rows at the end of ctx cached tokens, right-aligned causal mask; flops = causal "
                        "QK^T + PV",
            "configs": prefill_attn,
        },
        "c1_gemv": c1,
        "decode_sweep_fused_GBps": round(fused_gbs, 1),
        "decode_sweep_two_stage": {"GBps": round(two_gbs, 1), "us_per_step": round(two_ms * 1e3, 1),
                                   "routing": "scheme apply with HIF8_STATIC_FUSED_SINGLE_ROW=0 (the reference's "
                                              "routing): every projection static quant + GEMV; outputs equal"},
        "gemv_all_launches_GBps": round(all_gemv_gbs, 1),
        "gemm_per_layer": gemm_layer,
        "gemm_decoded_weights": {"routing": "HIF8_PREFILL_BF16_WEIGHTS=1: weights kept decoded to bf16 "
                                            "(2 B/element), soft_hif8_gemm_decoded_weight",
                                 **gemm_decoded},
        "ceilings": ceilings,
        "decode_ops": aux,
        "e2e_decode": e2e,
        "kernels": table,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
