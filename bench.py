"""Benchmark of the MI355X ring-attention path (one GPU).

Headline (BASELINE.json ``metric``): ring-prefill TFLOP/s at 32k on the Llama-3-8B
shape (config c3: S=32768 in 4 uneven domains [12288, 8192, 8192, 4096], 32 query /
8 KV heads, head_dim 128, bf16, causal).  One step = one full single-GPU ring replay
(every domain's ring steps: one block-kernel launch per non-empty (domain, source)
pair, each folding its source into the domain's running state, the last one writing
the output rows) through ``hcp_ring_prefill_replay``, inputs resident in HBM.  ``value`` counts
algorithmic FLOPs of causal pairs only: 2 GEMMs x 2 x D x Hq x S(S+1)/2.

Also reported on the same line: paged decode GB/s (config c4) and the growth-sharded
decode Q-ring at c4's shape, KV staging gather GB/s and the staged 128k prefill (config
c5), the LSE merge GB/s, the c3 prefill with Striped and ZigZag positions, the KV
wire-frame pack, the block-direct transport of a KV chunk, the fused QKV + RoPE + KV
append, fp32 on the matrix cores (c1 and an 8k block), a roofline object for the
dominant kernel (the flash block kernel, from HIP events recorded by the replay
driver on its launch stream over the timed region) and the CPU baseline (the oracle's
op-for-op libtorch restatement of ring.rs timed on this host on a bounded sample).

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "hetero-cp-ringattn_amd")

METRIC = "ring-prefill TFLOP/s (% MFMA peak) at 32k; paged-decode GB/s (% HBM peak)"
PEAK_BF16_TFLOPS = 2516.6   # 256 CU x 2.4 GHz x 4096 FLOP/clk/CU (dense)
PEAK_HBM_GBS = 8000.0
PEAK_FP32_MFMA_TFLOPS = 157.3  # dense fp32 on the matrix cores

C2 = dict(name="c2", chunks=[4096, 2560, 1536], hq=16, hkv=2, d=128, seed=43)
C3 = dict(name="c3", chunks=[12288, 8192, 8192, 4096], hq=32, hkv=8, d=128, seed=44)
C4 = dict(batch=64, hq=32, hkv=8, d=128, bs=16, ctx=16384, chunks=[8192, 5120, 3072],
          pool_blocks=65536, seed=45)
C5 = dict(chunks=[21504, 13312, 18432, 23552, 24576, 9216, 8192, 12288], hq=32, hkv=8, d=128,
          bs=16, seed=46)
# The reference's own model heads (Qwen2-0.5B: 14 q / 2 kv heads, head dim 64,
# docs/2domain_mps_hip_scale_matrix.md) on c2's chunks and on c3's 32k 4-domain split.
QWEN64 = dict(name="qwen2_0p5b_d64", chunks=[4096, 2560, 1536], hq=14, hkv=2, d=64, seed=47)
QWEN64_32K = dict(name="qwen2_0p5b_d64_32k", chunks=[12288, 8192, 8192, 4096], hq=14, hkv=2, d=64, seed=47)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def load_pkg():
    spec = importlib.util.spec_from_file_location(
        "hcp_ring_amd", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["hcp_ring_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def causal_flops(seq: int, hq: int, d: int) -> float:
    return 2.0 * d * hq * seq * (seq + 1)


def synth_qkv(H, torch, seq, hq, hkv, d, seed):
    """Q [S,Hq,D], K/V [S,Hkv,D] bf16 drawn Q, K, V from one LCG stream on the device."""
    q = torch.empty(seq, hq, d, dtype=torch.bfloat16, device="cuda")
    k = torch.empty(seq, hkv, d, dtype=torch.bfloat16, device="cuda")
    v = torch.empty(seq, hkv, d, dtype=torch.bfloat16, device="cuda")
    off = 0
    for t in (q, k, v):
        H.synth_normals(seed, off, t.numel(), t)
        off += t.numel()
    return q, k, v


def lcg_permutation(seed: int, n: int):
    """Fisher-Yates over range(n) driven by the 64-bit LCG's open-interval uniforms."""
    a, c, mask = 6364136223846793005, 1442695040888963407, (1 << 64) - 1
    s = seed
    p = list(range(n))
    for i in range(n - 1, 0, -1):
        s = (s * a + c) & mask
        u = ((s >> 11) + 0.5) / float(1 << 53)
        j = int(u * (i + 1))
        p[i], p[j] = p[j], p[i]
    return p


def time_cuda(torch, fn, reps: int) -> float:
    """Mean ms per call between torch events on the current stream."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


# ------------------------------------------------------------------ c3 prefill ----
def bench_prefill(H, torch, steps: int, warmup: int, c=None, schedule: str = "auto", tensors=None):
    """One ring replay per step (``schedule`` "auto": the fused single launch; "per_step":
    one grouped launch per ring step), inputs resident in HBM.  Whole-step time from the
    wall clock between synchronisations, then the same steps again with HIP events
    around every block-kernel launch for the kernel's own average launch time."""
    c = c or C3
    seq = sum(c["chunks"])
    if tensors is None:
        tensors = synth_qkv(H, torch, seq, c["hq"], c["hkv"], c["d"], c["seed"])
    q, k, v = tensors
    qh, kh, vh = (x.permute(1, 0, 2) for x in (q, k, v))
    ws = torch.empty(max(H.replay_workspace_size(torch.bfloat16, c["hq"], c["hkv"], c["d"], c["chunks"],
                                                 schedule=schedule), 1), dtype=torch.uint8, device="cuda")
    out = torch.empty(c["hq"], seq, c["d"], dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(c["hq"], seq, dtype=torch.float32, device="cuda")
    step = lambda: H.ring_attention_replay(qh, kh, vh, c["chunks"], out=out, lse_out=lse, workspace=ws,
                                           schedule=schedule)
    tag = f"{c.get('name', 'c3')} prefill ({schedule})"
    log(f"{tag} warmup x{warmup}")
    for _ in range(warmup):
        step()
    path = H.last_path()
    torch.cuda.synchronize()
    # whole-step time without instrumentation (per-launch events add ~10 us between launches)
    log(f"{tag} timed x{steps}")
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    H.replay_timing(True)
    H.replay_timing_read()
    log(f"{tag} per-launch timing x{steps}")
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    tm = H.replay_timing_read()
    H.replay_timing(False)
    flops = causal_flops(seq, c["hq"], c["d"])
    ms_step = elapsed * 1e3 / steps
    tflops = flops / (ms_step * 1e-3) / 1e12
    blk_ms, blk_n = tm["block"]
    per_launch_flops = flops * steps / blk_n
    avg_blk_ms = blk_ms / blk_n
    achieved = per_launch_flops / (avg_blk_ms * 1e-3) / 1e12
    if path == "ring_fused":
        # compulsory traffic of the one launch: Q, K and V read once, output rows and LSE written
        blk_bytes = seq * (c["hq"] * c["d"] * 2 * 2 + 2 * c["hkv"] * c["d"] * 2 + c["hq"] * 4)
    else:
        blk_bytes = sum(b for _, _, b in block_launch_bytes(c))
    finite = bool(torch.isfinite(lse).all().item()) and bool(torch.isfinite(out.float()).all().item())
    del ws
    return dict(ms_step=ms_step, tflops=tflops, flops=flops, blk_launches=blk_n // steps, path=path,
                avg_blk_ms=avg_blk_ms, per_launch_flops=per_launch_flops, achieved=achieved, finite=finite,
                alg_bytes_per_launch=blk_bytes * steps // blk_n, tensors=tensors, out=out, lse=lse)


def trace_summary(H, torch, c, tensors, launches: int):
    """Traced fused launches of a prefill config (hcp_ring_trace_attach): per launch the
    library's statistics, and over all launches a least-squares fit of workgroup
    duration against the 128-key tiles it folds (intercept = the fixed cost of a work
    item, slope = the cost of one tile), plus the shader clock from s_memtime."""
    import numpy as np

    q, k, v = tensors
    qh, kh, vh = (x.permute(1, 0, 2) for x in (q, k, v))
    n = len(c["chunks"])
    need = H.trace_record_bytes(torch.bfloat16, c["hq"], c["hkv"], c["d"], c["chunks"])
    buf = torch.zeros(need, dtype=torch.uint8, device="cuda")
    stride = 16 + 2 * n
    durs, tiles, clocks, per_launch, home = [], [], [], [], []
    H.trace_attach(buf)
    try:
        for _ in range(launches):
            H.ring_attention_replay(qh, kh, vh, c["chunks"])
            doms, launch = H.trace_read()
            per_launch.append(launch)
            rec = buf.view(torch.int32).cpu().numpy().view(np.uint32).reshape(-1, stride).astype(np.uint64)
            t0 = rec[:, 0] | (rec[:, 1] << 32)
            t1 = rec[:, 2] | (rec[:, 3] << 32)
            c0 = rec[:, 4] | (rec[:, 5] << 32)
            c1 = rec[:, 6] | (rec[:, 7] << 32)
            durs.append((t1 - t0).astype(np.float64) / 100.0)  # us (100 MHz ticks)
            tiles.append(rec[:, 12].astype(np.float64))
            clocks.append(100.0 * (c1 - c0).astype(np.float64) / (t1 - t0).astype(np.float64))
            # record i is work item i; id mod 8 is the XCD whose L2 streams its head group
            home.append(((rec[:, 9] & 15) % 8) == (np.arange(len(rec)) % 8))
    finally:
        H.trace_attach(None)
    dur, til, clk = np.concatenate(durs), np.concatenate(tiles), np.concatenate(clocks)
    slope, icpt = np.polyfit(til, dur, 1)
    resid = dur - (icpt + slope * til)
    keys = ["span_ms", "busy_cu_ms", "idle_gap_cu_ms", "tail_cu_ms", "head_cu_ms", "clock_mhz", "wg_ms_mean"]
    mean = {k: round(float(np.mean([x[k] for x in per_launch])), 4) for k in keys}
    return {"launches": launches, "workgroups": int(per_launch[0]["workgroups"]), "cus": int(per_launch[0]["cus"]),
            "mean_per_launch": mean,
            "span_ms_per_launch": [round(x["span_ms"], 4) for x in per_launch],
            "fit_us": {"per_item": round(float(icpt), 2), "per_key_tile": round(float(slope), 3),
                       "resid_rms": round(float(np.sqrt(np.mean(resid ** 2))), 2)},
            "wg_us": {"min": round(float(dur.min()), 1), "mean": round(float(dur.mean()), 1),
                      "max": round(float(dur.max()), 1)},
            "key_tiles_per_wg": {"min": int(til.min()), "mean": round(float(til.mean()), 2), "max": int(til.max())},
            "items_on_home_xcd": round(float(np.concatenate(home).mean()), 4),
            "clock_mhz": {"p10": round(float(np.percentile(clk, 10)), 1), "median": round(float(np.median(clk)), 1),
                          "p90": round(float(np.percentile(clk, 90)), 1)}}


def prefill_summary(r):
    """JSON object of a prefill leg (TFLOP/s of the whole step, and of the block kernel
    from its own launch times)."""
    return {"value": round(r["tflops"], 1), "unit": "TFLOP/s", "ms_per_step": round(r["ms_step"], 4),
            "frac_mfma": round(r["tflops"] / PEAK_BF16_TFLOPS, 4), "kernel_path": r["path"],
            "launches_per_step": r["blk_launches"], "kernel_tflops": round(r["achieved"], 1),
            "finite": r["finite"]}


def bench_c2(H, torch, steps: int, warmup: int):
    """Config c2 (Qwen2.5-3B shape): S=8192 in [4096, 2560, 1536], 16 q / 2 kv heads, D=128,
    bf16, causal, seed 43 -- both schedules."""
    fused = bench_prefill(H, torch, steps, warmup, C2, "auto")
    per = bench_prefill(H, torch, steps, warmup, C2, "per_step", tensors=fused["tensors"])
    log(f"c2 prefill {fused['tflops']:.1f} TFLOP/s fused, {per['tflops']:.1f} per step")
    res = {"workload": "c2: S=8192 in [4096,2560,1536], 16q/2kv heads, D=128, bf16, causal",
           **prefill_summary(fused), "per_step": prefill_summary(per),
           "max_abs_diff_schedules": round((fused["out"].float() - per["out"].float()).abs().max().item(), 5)}
    del fused, per
    return res


def bench_qwen_d64(H, torch, steps: int, warmup: int, c=None):
    """Ring prefill with Qwen2-0.5B heads (14 q / 2 kv, D=64), bf16, causal, fused
    schedule, K/V token-major as the projection writes them; head dim 64 runs the
    half-width instantiation of the block kernel (the 128-dim tiles, MFMAs on the first
    64 dims only).  Default: S=8192 in [4096, 2560, 1536]."""
    c = c or QWEN64
    r = bench_prefill(H, torch, steps, warmup, c)
    log(f"{c['name']} {r['tflops']:.1f} TFLOP/s ({r['path']})")
    chunks = ",".join(str(x) for x in c["chunks"])
    res = {"workload": f"Qwen2-0.5B heads: S={sum(c['chunks'])} in [{chunks}], 14q/2kv heads, D=64, bf16, causal",
           **prefill_summary(r)}
    del r
    return res


def block_launch_bytes(c):
    """Algorithmic HBM bytes of every block-kernel launch of one replay step, in launch
    order (ring step by ring step, targets ascending): Q + K + V reads, plus the
    running fp32 state (O + LSE) written by a domain's first source, read and written
    by its middle sources, read by its last source, which writes the output rows
    (bf16) and the fp32 LSE instead."""
    n = len(c["chunks"])
    offs = [sum(c["chunks"][:i]) for i in range(n)]
    d, hq, hkv = c["d"], c["hq"], c["hkv"]
    srcs = {t: [(t - s) % n for s in range(n) if offs[(t - s) % n] <= offs[t] + c["chunks"][t] - 1] for t in range(n)}
    out = []
    for step in range(n):
        for t in range(n):
            src = (t - step) % n
            if src not in srcs[t]:
                continue
            i, last = srcs[t].index(src), len(srcs[t]) - 1
            rows = c["chunks"][t] * hq
            b = rows * d * 2 + 2 * c["chunks"][src] * hkv * d * 2
            b += rows * (d + 1) * 4 * ((i > 0) + (i < last))   # state read / write
            b += rows * (2 * d + 4) * (i == last)               # output rows + LSE
            out.append((t, src, b))
    return out


# ------------------------------------------------------------------ c3 merge ----
def bench_strategies(H, torch, tensors, steps: int, warmup: int):
    """c3 ring prefill with Striped and ZigZag positions (strategy.rs:53-110): the same
    causal FLOPs, rows in domain-major order.  "auto": K/V copied in position order,
    then one positions-mode launch over the sequence (per-row key limits); "per_step":
    one grouped launch per ring step with the running state in HBM."""
    c = C3
    seq = sum(c["chunks"])
    qh, kh, vh = (x.permute(1, 0, 2) for x in tensors)
    out = torch.empty(c["hq"], seq, c["d"], dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(c["hq"], seq, dtype=torch.float32, device="cuda")
    res = {}
    for strat in ("striped", "zigzag"):
        for sched in ("auto", "per_step"):
            ws = torch.empty(H.replay_workspace_size(torch.bfloat16, c["hq"], c["hkv"], c["d"], c["chunks"],
                                                     strategy=strat, schedule=sched), dtype=torch.uint8,
                             device="cuda")
            step = lambda: H.ring_attention_replay(qh, kh, vh, c["chunks"], out=out, lse_out=lse, workspace=ws,
                                                   strategy=strat, schedule=sched)
            for _ in range(warmup):
                step()
            log(f"c3 prefill ({strat}, {sched}) timed x{steps}")
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                step()
            torch.cuda.synchronize()
            ms = (time.perf_counter() - t0) * 1e3 / steps
            r = {"value": round(causal_flops(seq, c["hq"], c["d"]) / (ms * 1e-3) / 1e12, 1),
                 "unit": "TFLOP/s", "ms_per_step": round(ms, 4), "finite": bool(torch.isfinite(lse).all().item())}
            if sched == "auto":
                res[strat] = r
            else:
                res[strat]["per_step"] = r
            del ws
    return res


def bench_fp32(H, torch, steps: int, warmup: int):
    """fp32, the reference's CPU dtype: c1 (seq 1024 in [640, 384], 8 heads, D=64,
    causal) as a ring replay, and one causal 8192-token block (Llama-3-8B heads, 32 q /
    8 kv, D=128) on the fp32 matrix-core kernel and on the scalar kernel (an output not
    16-byte aligned sends it there), against the fp32 matrix-core peak."""
    res = {}
    chunks, hq, d = [640, 384], 8, 64
    seq = sum(chunks)
    g = torch.Generator(device="cuda").manual_seed(42)
    q, k, v = (torch.randn(hq, seq, d, device="cuda", generator=g) for _ in range(3))
    step = lambda: H.ring_attention_replay(q, k, v, chunks)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    res["c1_replay"] = {"ms_per_step": round(ms, 4), "path": H.last_path(),
                        "value": round(causal_flops(seq, hq, d) / (ms * 1e-3) / 1e12, 3), "unit": "TFLOP/s"}
    lq, hq, hkv, d = 8192, 32, 8, 128
    q = torch.randn(hq, lq, d, device="cuda", generator=g)
    k, v = (torch.randn(hkv, lq, d, device="cuda", generator=g) for _ in range(2))
    flops = causal_flops(lq, hq, d)
    for aligned in (True, False):
        buf = torch.empty(hq * lq * d + 4, dtype=torch.float32, device="cuda")
        o = (buf[:hq * lq * d] if aligned else buf[1:1 + hq * lq * d]).view(hq, lq, d)
        lse = torch.empty(hq, lq, dtype=torch.float32, device="cuda")
        f = lambda: H.block_partial(q, k, v, 0, 0, o=o, lse=lse)
        f()
        torch.cuda.synchronize()
        path = H.last_path()
        n = max(steps // (1 if aligned else 5), 1)
        log(f"fp32 8k block ({path}) timed x{n}")
        t0 = time.perf_counter()
        for _ in range(n):
            f()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / n
        tf = flops / (ms * 1e-3) / 1e12
        res["block_8k_" + path] = {"ms": round(ms, 3), "value": round(tf, 2), "unit": "TFLOP/s",
                                   "frac_fp32_mfma": round(tf / PEAK_FP32_MFMA_TFLOPS, 4)}
        del buf, o, lse
    res["workload"] = ("fp32: c1 ring replay; causal 8192-token block, 32 q / 8 kv heads, D=128, on the fp32 "
                       "matrix-core kernel and the scalar kernel")
    return res


def bench_wire(H, torch, tensors, steps: int, warmup: int):
    """Device-side packing of one c3 domain chunk (8192 tokens) into the reference's
    TCP frame payload (GQA-expanded fp32 K/V + int64 positions, tcp.rs:161-207) and
    unpacking it back to compact bf16."""
    c = C3
    _, k, v = tensors
    off, n = c["chunks"][0], c["chunks"][1]
    kh, vh = (x[off:off + n].permute(1, 0, 2) for x in (k, v))
    pos = torch.arange(off, off + n, dtype=torch.int64, device="cuda")
    hdr, payload = H.kv_frame_pack(kh, vh, 0, off, off + n, positions=pos, num_heads=c["hq"])
    desc, _ = H.kv_frame_parse(hdr)
    desc.num_kv_heads = c["hkv"]
    ko = torch.empty(c["hkv"], n, c["d"], dtype=torch.bfloat16, device="cuda")
    vo = torch.empty_like(ko)
    pack = lambda: H.lib().hcp_kv_frame_pack(H.ctypes.byref(desc), H.view(kh), H.view(vh), H._ptr(pos),
                                             H._ptr(payload), None)
    unpack = lambda: H.lib().hcp_kv_frame_unpack(H.ctypes.byref(desc), H._ptr(payload), H.view(ko), H.view(vo),
                                                 None, None)
    if pack() != 0 or unpack() != 0:
        raise RuntimeError(f"wire pack/unpack failed: {H.last_error()}")
    for _ in range(warmup):
        pack()
        unpack()
    log(f"wire pack/unpack timed x{steps}")
    t_pack = time_cuda(torch, pack, steps)
    t_unpack = time_cuda(torch, unpack, steps)
    ok = bool(torch.equal(ko, kh) and torch.equal(vo, vh))
    compact = 2 * c["hkv"] * n * c["d"] * 2
    wire = payload.numel()
    return {"workload": f"c3 domain-1 chunk ({n} tokens): bf16 [8, L, 128] K/V -> reference TCP payload "
                        f"(fp32, expanded to 32 heads, + int64 positions) and back",
            "pack_gbs": round((compact + wire) / (t_pack * 1e-3) / 1e9, 1),
            "unpack_gbs": round((wire // 4 + compact) / (t_unpack * 1e-3) / 1e9, 1),
            "unit": "GB/s", "pack_ms": round(t_pack, 4), "unpack_ms": round(t_unpack, 4),
            "payload_bytes": wire, "round_trip_bit_exact": ok}


def bench_qkv(H, torch, steps: int, warmup: int):
    """Fused QKV projection + RoPE + paged KV append for the Llama-3-8B layer shape
    (hidden 4096, 32 q / 8 kv heads, D = 128) over one c3 domain chunk of 12288 tokens,
    beside torch.matmul (the vendor GEMM) of the same concatenated projection alone."""
    c = C3
    tokens, hidden = c["chunks"][0], 4096
    hq, hkv, d = c["hq"], c["hkv"], c["d"]
    n_feat = (hq + 2 * hkv) * d
    x = torch.empty(tokens, hidden, dtype=torch.bfloat16, device="cuda")
    w = torch.empty(n_feat, hidden, dtype=torch.bfloat16, device="cuda")
    H.synth_normals(47, 0, x.numel(), x)
    H.synth_normals(47, x.numel(), w.numel(), w)
    w.mul_(1.0 / math.sqrt(hidden))
    wq, wk, wv = w[: hq * d], w[hq * d: (hq + hkv) * d], w[(hq + hkv) * d:]
    table = H.rope_table(d, 32768, 500000.0)
    pos = torch.arange(tokens, dtype=torch.int64, device="cuda")
    bs = 16
    nb = tokens // bs + 8
    pool = torch.empty(2, nb, bs, hkv, d, dtype=torch.bfloat16, device="cuda")
    blocks = torch.arange(tokens // bs, dtype=torch.int32, device="cuda")
    q = torch.empty(hq, tokens, d, dtype=torch.bfloat16, device="cuda")
    run = lambda: H.qkv_rope_project_paged(x, wq, wk, wv, hq, hkv, d, pool, blocks, 0, 0, positions=pos,
                                           table=table, q_out=q)
    for _ in range(warmup):
        run()
    log(f"qkv+rope timed x{steps}")
    ms = time_cuda(torch, run, steps)
    y = torch.empty(tokens, n_feat, dtype=torch.bfloat16, device="cuda")
    gemm = lambda: torch.matmul(x, w.t(), out=y)
    for _ in range(warmup):
        gemm()
    ms_gemm = time_cuda(torch, gemm, steps)
    flops = 2.0 * tokens * hidden * n_feat
    return {"workload": f"Llama-3-8B QKV: {tokens} tokens x hidden {hidden} -> {hq}q/{hkv}kv heads x {d}, "
                        "bias-free, RoPE (theta 5e5), k/v appended to a bs=16 paged pool",
            "value": round(flops / (ms * 1e-3) / 1e12, 1), "unit": "TFLOP/s", "ms": round(ms, 4),
            "frac_mfma": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "vendor_gemm_only_tflops": round(flops / (ms_gemm * 1e-3) / 1e12, 1),
            "finite": bool(torch.isfinite(q.float()).all().item())}


def bench_merge(H, torch, steps: int, warmup: int):
    """The LSE merge kernel (hcp_ring_lse_merge) on the c3 shapes: per target domain,
    its non-empty ring partials (o [Hq, L, D] + lse [Hq, L] fp32) -> bf16 rows + fp32
    LSE.  The ring replay itself folds sources as they arrive, so this is the merge
    entry point's own measurement (the decode path uses it after every chunk)."""
    c = C3
    n = len(c["chunks"])
    offs = [sum(c["chunks"][:i]) for i in range(n)]
    jobs, mbytes, off = [], 0, 0
    for t in range(n):
        parts = sum(1 for s_ in range(n) if offs[s_] <= offs[t] + c["chunks"][t] - 1)
        L = c["chunks"][t]
        os_ = [torch.empty(c["hq"], L, c["d"], dtype=torch.float32, device="cuda") for _ in range(parts)]
        ls_ = [torch.empty(c["hq"], L, dtype=torch.float32, device="cuda") for _ in range(parts)]
        for x in os_ + ls_:
            H.synth_normals(c["seed"] + 1, off, x.numel(), x)
            off += x.numel()
        out = torch.empty(c["hq"], L, c["d"], dtype=torch.bfloat16, device="cuda")
        lse = torch.empty(c["hq"], L, dtype=torch.float32, device="cuda")
        jobs.append((os_, ls_, out, lse))
        mbytes += c["hq"] * L * (parts * (4 * c["d"] + 4) + 2 * c["d"] + 4)

    def step():
        for os_, ls_, out, lse in jobs:
            H.lse_merge(os_, ls_, out=out, lse_out=lse)

    for _ in range(warmup):
        step()
    ms = time_cuda(torch, step, steps)
    res = dict(merge_ms=ms, merge_gbs=mbytes / (ms * 1e-3) / 1e9, merge_bytes=mbytes)
    del jobs
    return res


# ------------------------------------------------------------------ c4 decode ----
def bench_decode(H, torch, steps: int, warmup: int):
    c = C4
    nb, bs, hkv, d = c["pool_blocks"], c["bs"], c["hkv"], c["d"]
    q = torch.empty(c["batch"], c["hq"], d, dtype=torch.bfloat16, device="cuda")
    pool = torch.empty(2, nb, bs, hkv, d, dtype=torch.bfloat16, device="cuda")
    H.synth_normals(c["seed"], 0, q.numel(), q)
    H.synth_normals(c["seed"], q.numel(), pool.numel(), pool)
    perm = lcg_permutation(c["seed"], nb)
    per_seq = c["ctx"] // bs
    tables = torch.tensor(perm[: c["batch"] * per_seq], dtype=torch.int32, device="cuda").view(c["batch"], per_seq)
    bounds, acc = [], 0
    for L in c["chunks"]:
        bounds.append((acc, acc + L))
        acc += L
    outs = [(torch.empty(c["batch"], c["hq"], d, dtype=torch.float32, device="cuda"),
             torch.empty(c["batch"], c["hq"], dtype=torch.float32, device="cuda")) for _ in bounds]
    wss = [torch.empty(max(H.decode_workspace_size(q, pool, tables, t0, t1), 1), dtype=torch.uint8, device="cuda")
           for t0, t1 in bounds]
    final = torch.empty(c["batch"], c["hq"], d, dtype=torch.bfloat16, device="cuda")
    final_lse = torch.empty(c["batch"], c["hq"], dtype=torch.float32, device="cuda")

    def chunk(i):
        t0, t1 = bounds[i]
        H.decode_local_compact_partial(q, pool, tables, t0, t1, workspace=wss[i], o=outs[i][0], lse=outs[i][1])

    def step():
        for i in range(len(bounds)):
            chunk(i)
        # per-chunk partials merged across domains: rows = batch*Hq, one token each
        H.lse_merge([o.view(-1, 1, d) for o, _ in outs],
                    [l.view(-1, 1) for _, l in outs], out=final.view(-1, 1, d), lse_out=final_lse.view(-1, 1))

    log(f"c4 decode warmup x{warmup}")
    for _ in range(warmup):
        step()
    log(f"c4 decode timed x{steps}")
    ms_step = time_cuda(torch, step, steps)
    kv_bytes = 2 * c["batch"] * c["ctx"] * hkv * d * 2
    alg_bytes = kv_bytes + q.numel() * 2 + c["batch"] * c["hq"] * (d + 1) * 4 * len(bounds) \
        + tables.numel() * 4 + final.numel() * 2
    # dominant kernel: the chunk-0 decode call (8192 keys of each sequence)
    ms_c0 = time_cuda(torch, lambda: chunk(0), steps)
    c0_bytes = 2 * c["batch"] * c["chunks"][0] * hkv * d * 2
    res = dict(ms_step=ms_step, gbs=alg_bytes / (ms_step * 1e-3) / 1e9, bytes=alg_bytes,
               chunk0_ms=ms_c0, chunk0_gbs=c0_bytes / (ms_c0 * 1e-3) / 1e9,
               finite=bool(torch.isfinite(final.float()).all().item()))
    del pool
    return res


def bench_decode_ring(H, torch, steps: int, warmup: int):
    """One decode step of the Q-ring with growth sharding (hcp_decode_ring_replay,
    ring.rs:665-818, owner rule ring.rs:1930-1936) at c4's shape: 64 sequences of 16384
    tokens, the first 16288 prefilled over c4's three domains (the last domain's chunk
    96 shorter), the last 96 decode tokens each in its owner's shard (p mod 3).  Each
    domain's shard is its own permuted bs=16 block table; one replay runs the paged
    decode over every shard and the journey-order merge.  Synthetic K/V: the timing and
    the bytes, not the values, are what this leg measures (parity: the GPU tests)."""
    c = C4
    b, hq, hkv, d, bs = c["batch"], c["hq"], c["hkv"], c["d"], c["bs"]
    n = len(c["chunks"])
    dec = 96
    prefill = c["ctx"] - dec
    chunks = list(c["chunks"])
    chunks[-1] -= dec
    lens = [chunks[dom] + sum(1 for p in range(prefill, c["ctx"]) if p % n == dom) for dom in range(n)]
    nblk = [-(-L // bs) for L in lens]
    nb = b * sum(nblk) + 1
    q = torch.empty(b, hq, d, dtype=torch.bfloat16, device="cuda")
    pool = torch.empty(2, nb, bs, hkv, d, dtype=torch.bfloat16, device="cuda")
    H.synth_normals(c["seed"] + 7, 0, q.numel(), q)
    H.synth_normals(c["seed"] + 7, q.numel(), pool.numel(), pool)
    perm = lcg_permutation(c["seed"] + 7, nb)
    shards, cur = [], 0
    for dom in range(n):
        tab = torch.tensor(perm[cur: cur + b * nblk[dom]], dtype=torch.int32, device="cuda").view(b, nblk[dom])
        cur += b * nblk[dom]
        shards.append((tab, torch.full((b,), lens[dom], dtype=torch.int32, device="cuda"), lens[dom]))
    out = torch.empty(b, hq, d, dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(b, hq, dtype=torch.float32, device="cuda")
    # the replay's workspace (split partials and the N domain partials), allocated once
    ws = torch.empty(max(H.decode_ring_workspace_size(q, pool, shards), 1), dtype=torch.uint8, device="cuda")

    def step():
        H.decode_ring_replay(q, pool, shards, 0, out=out, lse_out=lse, workspace=ws)

    log(f"decode ring warmup x{warmup}")
    for _ in range(warmup):
        step()
    log(f"decode ring timed x{steps}")
    ms = time_cuda(torch, step, steps)
    kv_bytes = 2 * b * sum(lens) * hkv * d * 2
    alg = kv_bytes + q.numel() * 2 + 2 * n * b * hq * (d + 1) * 4 + b * sum(nblk) * 4 + out.numel() * 2 + lse.numel() * 4
    gbs = alg / (ms * 1e-3) / 1e9
    res = dict(workload=f"f1 decode Q-ring: B={b}, ctx {c['ctx']} growth-sharded over {n} domains "
                        f"(prefill {chunks}, {dec} decode tokens by owner p mod {n}), {hq}q/{hkv}kv, D={d}, bf16, "
                        f"bs={bs}; one hcp_decode_ring_replay (paged decode per shard + journey-order merge)",
               value=round(gbs, 1), unit="GB/s", ms_per_step=round(ms, 4), frac_hbm=round(gbs / PEAK_HBM_GBS, 4),
               bytes=alg, finite=bool(torch.isfinite(out.float()).all().item()))
    del pool
    return res


def bench_block_transport(H, torch, steps: int, warmup: int):
    """The block-direct transport (block_transport.rs:36-126) moving one c3 domain-1 K/V
    chunk (8192 tokens, 8 KV heads, D=128, bf16: K and V in one [2, 8, 8192, 128]
    block, 32 MiB) between a linked agent pair on this GPU: per step one
    submit_transfer (an async device copy) and host polls until the receiver reports
    the completion.  GB/s counts the block's bytes once (the bytes on the wire)."""
    src = torch.empty(2, 8, 8192, 128, dtype=torch.bfloat16, device="cuda")
    H.synth_normals(C3["seed"] + 3, 0, src.numel(), src)
    dst = torch.zeros_like(src)
    sender, receiver = H.BlockAgent.pair("domain-0", "domain-1")
    try:
        dst_id, _ = receiver.register_block(dst)
        src_id, _ = sender.register_block(src)
        receiver.load_remote_metadata(sender.local_metadata())
        sender.load_remote_metadata(receiver.local_metadata())
        remote = sender.remote_desc("domain-1", dst_id)

        def step():
            sender.submit_transfer(src_id, remote)
            while not receiver.poll_transfers():
                pass

        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        exact = bool(torch.equal(dst.view(torch.int16), src.view(torch.int16)))
        sent, _ = sender.wire_bytes()
    finally:
        sender.destroy()
        receiver.destroy()
    nbytes = src.numel() * 2
    return dict(workload="f3 block-direct transport: one c3 domain-1 K/V chunk (8192 tokens, 8 kv heads, D=128, "
                         "bf16, 32 MiB) per step, submit_transfer + receiver polls until completion",
                value=round(nbytes / (ms * 1e-3) / 1e9, 1), unit="GB/s", ms_per_step=round(ms, 4), bytes=nbytes,
                bit_exact=exact, wire_bytes_sent=int(sent))


# ------------------------------------------------------------------ c5 staging ----
def bench_staged(H, torch, steps: int, warmup: int, full_prefill: bool = True):
    c = C5
    seq, hkv, d, bs = sum(c["chunks"]), c["hkv"], c["d"], c["bs"]
    q, k, v = synth_qkv(H, torch, seq, c["hq"], hkv, d, c["seed"])
    nb = seq // bs
    perm = lcg_permutation(42, nb)
    table = torch.tensor(perm, dtype=torch.int32, device="cuda")
    pool = torch.zeros(2, nb, bs, hkv, d, dtype=torch.bfloat16, device="cuda")
    H.paged_kv_scatter(pool, table, 0, 0, seq, k.permute(1, 0, 2), v.permute(1, 0, 2))
    offs = [sum(c["chunks"][:i]) for i in range(len(c["chunks"]))]
    stage_k = torch.empty(hkv, seq, d, dtype=torch.bfloat16, device="cuda")
    stage_v = torch.empty(hkv, seq, d, dtype=torch.bfloat16, device="cuda")

    ranges = [(table, 0, o, o + L, stage_k[:, o:o + L], stage_v[:, o:o + L]) for o, L in zip(offs, c["chunks"])]

    # every domain's chunk staged by one batched launch (8 ranges); descriptors built once
    gather_all = H.paged_gather_plan(pool, ranges)

    for _ in range(warmup):
        gather_all()
    ms = time_cuda(torch, gather_all, steps)
    gbytes = 2 * seq * hkv * d * 2 * 2
    exact = bool(torch.equal(stage_k.view(torch.int16), k.permute(1, 0, 2).contiguous().view(torch.int16))) and \
        bool(torch.equal(stage_v.view(torch.int16), v.permute(1, 0, 2).contiguous().view(torch.int16)))
    # the reverse direction (KvCache::update): scatter the whole sequence back into the pool
    kh, vh = stage_k, stage_v
    scatter = lambda: H.paged_kv_scatter(pool, table, 0, 0, seq, kh, vh)
    for _ in range(warmup):
        scatter()
    ms_s = time_cuda(torch, scatter, steps)
    res = dict(gather_ms=ms, gather_gbs=gbytes / (ms * 1e-3) / 1e9, gather_bytes=gbytes, bit_exact=exact,
               scatter_ms=ms_s, scatter_gbs=gbytes / (ms_s * 1e-3) / 1e9)
    del stage_k, stage_v
    if full_prefill:
        ws = torch.empty(H.replay_workspace_size(torch.bfloat16, c["hq"], hkv, d, c["chunks"], paged=True),
                         dtype=torch.uint8, device="cuda")
        out = torch.empty(c["hq"], seq, d, dtype=torch.bfloat16, device="cuda")
        lse = torch.empty(c["hq"], seq, dtype=torch.float32, device="cuda")
        run = lambda: H.ring_attention_replay_paged(q.permute(1, 0, 2), pool, table, c["chunks"], out=out,
                                                    lse_out=lse, workspace=ws)
        run()
        path = H.last_path()
        reps = 3
        ms_p = time_cuda(torch, run, reps)
        res.update(prefill_ms=ms_p, prefill_tflops=causal_flops(seq, c["hq"], d) / (ms_p * 1e-3) / 1e12,
                   prefill_path=path,
                   prefill_finite=bool(torch.isfinite(lse).all().item()) and bool(torch.isfinite(out.float()).all().item()))
        # a few rows at domain boundaries against the f64 closed form (the parity tests check more)
        rows = [offs[1] - 1, offs[4], offs[7], seq - 1]
        e_o, e_l = sampled_rows_error(q, k, v, out, lse, rows)
        res.update(sampled_rows=rows, sampled_err_out=e_o, sampled_err_lse=e_l)
        del ws
    return res


def sampled_rows_error(q, k, v, out, lse, rows):
    """Max |out - f64| and |lse - f64| over query rows `rows` of a causal vanilla replay
    (q [S, Hq, D], k/v [S, Hkv, D]; out [Hq, S, D], lse [Hq, S]), all heads."""
    import numpy as np
    hq, hkv, d = q.shape[1], k.shape[1], q.shape[2]
    rep = hq // hkv
    k64 = k.double().cpu().numpy()
    v64 = v.double().cpu().numpy()
    e_o = e_l = 0.0
    for r in rows:
        qr = q[r].double().cpu().numpy()
        go = out[:, r].double().cpu().numpy()
        gl = lse[:, r].double().cpu().numpy()
        for g in range(hkv):
            s_ = qr[g * rep:(g + 1) * rep] @ k64[: r + 1, g].T / math.sqrt(d)
            m = s_.max(axis=1, keepdims=True)
            w = np.exp(s_ - m)
            den = w.sum(axis=1, keepdims=True)
            o = (w @ v64[: r + 1, g]) / den
            e_o = max(e_o, float(np.abs(go[g * rep:(g + 1) * rep] - o).max()))
            e_l = max(e_l, float(np.abs(gl[g * rep:(g + 1) * rep] - (m + np.log(den))[:, 0]).max()))
    return round(e_o, 6), round(e_l, 7)


# ------------------------------------------------------------------ CPU baseline ----
def cpu_model() -> str:
    """The host CPU's model string (/proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(torch, tensors, budget_s: float = 10.0):
    """The oracle's op-for-op libtorch restatement of ring.rs (ring_attention driver,
    process_kv_block folds, bf16 state, 2048 tiling, GQA-expand copies) on this host:
    whole target domains of c3, in order 0, 1, 2, 3, until the budget is spent (at
    least one).  value = algorithmic causal FLOPs of the completed domains / time."""
    sys.path.insert(0, ROOT)
    from oracle import tch_ring

    c = C3
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    q, k, v = tensors
    n = len(c["chunks"])
    offs = [sum(c["chunks"][:i]) for i in range(n)]
    rep = c["hq"] // c["hkv"]
    scale = 1 / math.sqrt(c["d"])
    qh = q.permute(1, 0, 2).unsqueeze(0).cpu()
    kx = tch_ring.repeat_kv_heads(k.permute(1, 0, 2).unsqueeze(0).cpu(), rep)
    vx = tch_ring.repeat_kv_heads(v.permute(1, 0, 2).unsqueeze(0).cpu(), rep)
    sent = [tch_ring.local_micro_blocks(kx[:, :, o:o + L], vx[:, :, o:o + L], o, n)
            for o, L in zip(offs, c["chunks"])]
    flops, t_total, done = 0.0, 0.0, []
    for d in range(n):
        o, L = offs[d], c["chunks"][d]
        rounds = [sent[(d - 1 - r) % n] for r in range(n - 1)]
        t0 = time.perf_counter()
        tch_ring.ring_attention(scale, qh[:, :, o:o + L], kx[:, :, o:o + L], vx[:, :, o:o + L],
                                torch.arange(o, o + L), o, n, rounds)
        t_total += time.perf_counter() - t0
        # causal pairs of rows o..o+L-1: sum (p+1)
        flops += 4.0 * c["d"] * c["hq"] * (L * o + L * (L + 1) / 2)
        done.append(d)
        log(f"cpu baseline domain {d}: {t_total:.1f}s")
        if t_total >= budget_s:
            break
    return dict(value=flops / t_total / 1e12, unit="TFLOP/s", cores=torch.get_num_threads(), kind="port",
                nproc=os.cpu_count(), cpu_model=cpu_model(),
                sample=f"c3 ring_attention of target domains {done} (of 4), op-for-op libtorch restatement of "
                       f"ring.rs:861-1398 (bf16 state, 2048 q/kv tiles, GQA-expanded K/V), {t_total:.1f} s; "
                       f"algorithmic causal FLOPs of those domains / time")


def profiled_traffic(name: str):
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3 PMC
    summary (FETCH_SIZE and WRITE_SIZE passes scaled by a plain-copy calibration);
    None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def copy_calibration():
    """Three copies of 1 GiB by torch's plain copy kernel: the PMC counters of these
    dispatches convert FETCH_SIZE / WRITE_SIZE readings into bytes."""
    import torch

    a = torch.empty(1 << 28, dtype=torch.float32, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_dispatch": a.numel() * 4, "dispatches": 3}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # The first few c3 steps on a fresh box run 2-7% slower than later ones (measured in
    # the kernel trace); the default warmup covers them.
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="headline prefill only")
    ap.add_argument("--only-prefill", action="store_true", help="c3 prefill only, no CPU leg (profiling)")
    ap.add_argument("--leg", choices=["c2", "c3", "qwen64", "qwen64_32k", "strategies", "fp32", "merge", "staging",
                                      "decode_ring", "block_transport"],
                    default=None,
                    help="run one prefill leg alone and print its JSON object (profiling)")
    ap.add_argument("--trace", action="store_true",
                    help="with --leg: also run traced launches (per-workgroup records) and summarise them")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run three plain 1 GiB device copies (calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.only_prefill:
        args.no_extra = args.no_cpu = True
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the ring is replayed on a single MI355X "
              "(multi-GPU rings are a design note, not part of this build); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    import torch

    H = load_pkg()
    torch.cuda.set_device(0)
    log(f"device {torch.cuda.get_device_name(0)}")
    if args.leg in ("qwen64", "qwen64_32k"):
        c = QWEN64 if args.leg == "qwen64" else QWEN64_32K
        print(json.dumps({"leg": args.leg, **bench_qwen_d64(H, torch, args.steps, args.warmup, c)}), flush=True)
        return
    if args.leg == "staging":
        g = bench_staged(H, torch, args.steps, args.warmup, full_prefill=False)
        print(json.dumps({"leg": "staging", "value": round(g["scatter_gbs"], 1), "unit": "GB/s",
                          "ms_per_step": round(g["scatter_ms"], 4), "gather_gbs": round(g["gather_gbs"], 1),
                          "bit_exact": g["bit_exact"]}), flush=True)
        return
    if args.leg == "merge":
        m = bench_merge(H, torch, args.steps, args.warmup)
        print(json.dumps({"leg": "merge", "value": round(m["merge_gbs"], 1), "unit": "GB/s",
                          "ms_per_step": round(m["merge_ms"], 4), "frac_hbm": round(m["merge_gbs"] / PEAK_HBM_GBS, 4),
                          "bytes": m["merge_bytes"]}), flush=True)
        return
    if args.leg == "block_transport":
        print(json.dumps({"leg": "block_transport", **bench_block_transport(H, torch, args.steps, args.warmup)}),
              flush=True)
        return
    if args.leg == "decode_ring":
        print(json.dumps({"leg": "decode_ring", **bench_decode_ring(H, torch, args.steps, args.warmup)}), flush=True)
        return
    if args.leg == "fp32":
        print(json.dumps({"leg": "fp32", **bench_fp32(H, torch, args.steps, args.warmup)}), flush=True)
        return
    if args.leg == "strategies":
        tensors = synth_qkv(H, torch, sum(C3["chunks"]), C3["hq"], C3["hkv"], C3["d"], C3["seed"])
        print(json.dumps({"leg": "strategies", **bench_strategies(H, torch, tensors, args.steps, args.warmup)}),
              flush=True)
        return
    if args.leg is not None:
        c = {"c2": C2, "c3": C3}[args.leg]
        r = bench_prefill(H, torch, args.steps, args.warmup, c)
        out = {"leg": args.leg, **prefill_summary(r)}
        if args.trace:
            out["trace"] = trace_summary(H, torch, c, r["tensors"], launches=args.steps)
        print(json.dumps(out), flush=True)
        return
    pre = bench_prefill(H, torch, args.steps, args.warmup)
    log(f"c3 prefill {pre['tflops']:.1f} TFLOP/s ({pre['ms_step']:.3f} ms/step, {pre['path']})")
    extra = {}

    def guarded(keys, fn):
        # One extra leg: a failure is reported inside the JSON line under the leg's keys
        # (and logged), so it cannot take the headline figure with it.
        try:
            extra.update(fn())
        except Exception as e:  # noqa: BLE001
            msg = f"{type(e).__name__}: {e}"
            log(f"extra leg {'/'.join(keys)} failed: {msg}")
            extra.update({k: {"error": msg} for k in keys})

    def leg_per_step():
        # the same c3 replay under the per-step schedule (one grouped launch per ring step)
        per = bench_prefill(H, torch, args.steps, args.warmup, schedule="per_step", tensors=pre["tensors"])
        log(f"c3 prefill per step {per['tflops']:.1f} TFLOP/s")
        diff = (per["out"].float() - pre["out"].float()).abs().max().item()
        return dict(c3_per_step=dict(workload="c3 with schedule per_step (one grouped launch per ring step, fp32 "
                                              "state in HBM between steps)", **prefill_summary(per),
                                     max_abs_diff_vs_fused=round(diff, 5)))

    def leg_decode():
        dec = bench_decode(H, torch, args.steps, args.warmup)
        log(f"c4 decode {dec['gbs']:.1f} GB/s")
        return dict(paged_decode={"workload": "c4: B=64, ctx 16384 in [8192,5120,3072], 32q/8kv, D=128, bf16, bs=16",
                                  "value": round(dec["gbs"], 1), "unit": "GB/s",
                                  "ms_per_step": round(dec["ms_step"], 4),
                                  "frac_hbm": round(dec["gbs"] / PEAK_HBM_GBS, 4), "bytes": dec["bytes"],
                                  "chunk0_kernel_gbs": round(dec["chunk0_gbs"], 1), "finite": dec["finite"]})

    def leg_staging():
        stg = bench_staged(H, torch, args.steps, args.warmup)
        log(f"c5 gather {stg['gather_gbs']:.1f} GB/s, prefill {stg.get('prefill_tflops', 0):.1f} TFLOP/s")
        return dict(
            kv_staging={"workload": "c5: gather of all 8 chunks (131072 tokens, 8 kv heads, D=128, bf16) from a "
                                    "permuted bs=16 block pool",
                        "value": round(stg["gather_gbs"], 1), "unit": "GB/s", "ms": round(stg["gather_ms"], 4),
                        "frac_hbm": round(stg["gather_gbs"] / PEAK_HBM_GBS, 4), "bytes": stg["gather_bytes"],
                        "bit_exact": stg["bit_exact"], "scatter_gbs": round(stg["scatter_gbs"], 1),
                        "scatter_ms": round(stg["scatter_ms"], 4)},
            staged_prefill_128k={"workload": "c5: every chunk gathered from the paged pool (one batched launch), "
                                             "then the fused ring over 131072 tokens in 8 domains",
                                 "value": round(stg.get("prefill_tflops", 0.0), 1), "unit": "TFLOP/s",
                                 "ms": round(stg.get("prefill_ms", 0.0), 3),
                                 "frac_mfma": round(stg.get("prefill_tflops", 0.0) / PEAK_BF16_TFLOPS, 4),
                                 "kernel_path": stg.get("prefill_path"), "finite": stg.get("prefill_finite"),
                                 "sampled_rows": stg.get("sampled_rows"),
                                 "sampled_max_abs_err_out": stg.get("sampled_err_out"),
                                 "sampled_max_abs_err_lse": stg.get("sampled_err_lse")})

    def leg_merge():
        mrg = bench_merge(H, torch, args.steps, args.warmup)
        log(f"c3 lse merge {mrg['merge_gbs']:.1f} GB/s")
        return dict(lse_merge={"workload": "c3 ring partials of the 4 target domains (10 x [32, L, 128] fp32 + LSE) "
                                           "-> bf16 rows + fp32 LSE, one hcp_ring_lse_merge per domain",
                               "value": round(mrg["merge_gbs"], 1), "unit": "GB/s",
                               "ms_per_step": round(mrg["merge_ms"], 4),
                               "frac_hbm": round(mrg["merge_gbs"] / PEAK_HBM_GBS, 4), "bytes": mrg["merge_bytes"]})

    def leg_strategies():
        strat = bench_strategies(H, torch, pre["tensors"], args.steps, args.warmup)
        log(f"c3 strategies {strat}")
        return dict(strategies=dict(workload="c3 ring prefill with Striped / ZigZag positions (same causal FLOPs)",
                                    **strat))

    def leg_logged(key, fn):
        def run():
            r = fn()
            log(f"{key} {r}")
            return {key: r}
        return run

    if not args.no_extra:
        guarded(["c3_per_step"], leg_per_step)
        guarded(["c2_prefill"], leg_logged("c2_prefill", lambda: bench_c2(H, torch, args.steps, args.warmup)))
        guarded(["qwen2_0p5b_d64_8k"], leg_logged("qwen2_0p5b_d64_8k",
                                                  lambda: bench_qwen_d64(H, torch, args.steps, args.warmup)))
        guarded(["qwen2_0p5b_d64_32k"], leg_logged("qwen2_0p5b_d64_32k",
                                                   lambda: bench_qwen_d64(H, torch, args.steps, args.warmup,
                                                                          QWEN64_32K)))
        guarded(["paged_decode"], leg_decode)
        guarded(["decode_ring"], leg_logged("decode_ring", lambda: bench_decode_ring(H, torch, args.steps,
                                                                                   args.warmup)))
        guarded(["kv_staging", "staged_prefill_128k"], leg_staging)
        guarded(["lse_merge"], leg_merge)
        guarded(["strategies"], leg_strategies)
        guarded(["kv_frame"], leg_logged("kv_frame", lambda: bench_wire(H, torch, pre["tensors"], args.steps,
                                                                        args.warmup)))
        guarded(["block_transport"], leg_logged("block_transport", lambda: bench_block_transport(H, torch, args.steps,
                                                                                              args.warmup)))
        guarded(["qkv_rope"], leg_logged("qkv_rope", lambda: bench_qkv(H, torch, args.steps, args.warmup)))
        guarded(["fp32"], leg_logged("fp32", lambda: bench_fp32(H, torch, args.steps, args.warmup)))
    cpu = None
    if not args.no_cpu:
        try:
            cpu = cpu_baseline(torch, pre["tensors"])
            log(f"cpu baseline {cpu['value']:.4f} TFLOP/s on {cpu['cores']} threads")
        except Exception as e:  # noqa: BLE001 -- reported in the line, like a failed extra leg
            cpu = {"error": f"{type(e).__name__}: {e}"}
            log(f"cpu baseline failed: {cpu['error']}")
    line = {
        "metric": METRIC,
        "value": round(pre["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pre["ms_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (LCG + Box-Muller normals, seed 44, generated on the device)",
        "config": {"workload": "c3_llama3_8b_ring_prefill_32k", "chunks": C3["chunks"], "num_q_heads": C3["hq"],
                   "num_kv_heads": C3["hkv"], "head_dim": C3["d"], "causal": True,
                   "flops_per_step": pre["flops"], "frac_mfma_peak": round(pre["tflops"] / PEAK_BF16_TFLOPS, 4)},
        "roofline": {"bound": "mfma",
                     "kernel": "flash_ring_kernel" if pre["path"] == "ring_fused" else "flash_block_pingpong_kernel",
                     "achieved": round(pre["achieved"], 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(pre["achieved"] / PEAK_BF16_TFLOPS, 4),
                     "traffic": profiled_traffic("flash_ring_kernel_c3_prefill.md" if pre["path"] == "ring_fused"
                                                 else "flash_block_kernel_c3_prefill.md"),
                     "algorithmic_bytes_per_launch": pre["alg_bytes_per_launch"],
                     "launches_per_step": pre["blk_launches"], "avg_launch_ms": round(pre["avg_blk_ms"], 4),
                     "flops_per_launch": pre["per_launch_flops"]},
        "cpu_baseline": cpu,
        "finite": pre["finite"],
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
