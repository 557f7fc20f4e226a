"""Decode-step benchmark of the fp8 KV path on one MI355X.

A step is one pass of the hot path over one batch: the QK-norm + RoPE + fp8 append of the step's token for every
sequence, then split-K decode attention over the paged fp8 cache, both in one launch (nc_decode_step_fp8; with
--two-launch, nc_qk_norm_rope_append_fp8 then nc_decode_attn_fp8, the same bits). Default workload: the headline "bs64 ctx8K" (B = 64, 16 query / 4 KV heads, 8192
cached tokens + the step's, 16-token pages under a random-permutation block table, 1% outliers at 8 sigma),
synthetic seeded data resident in HBM before the timed region.

value = algorithmic HBM bytes of the step / step time (GB/s). Attention bytes per (sequence, KV head):
(n + 1) * 264 (fp8 K + V and two fp32 scales per key) + G * 128 * 2 * 2 (q in, out) + ceil((n + 1) / 16) * 4
(block table); the append adds 2 Hkv * 256 read (the token's k and v rows; its q row is the attention's q read) and
Hkv * 264 written (codes and scales) per token.

    python bench.py [--steps K] [--warmup W] [--workload c3u|c3|c2|c1|c4|c5|ve|fa] [--workers W] [--cpu-seqs S]
                    [--no-e2e] [--two-launch]

A decode workload's line also carries the metric's second half, `decode_tokens_per_s`: config 5 end to end
(below), unless --no-e2e.

--workload c4 times the chunked-prefill step instead (TFLOP/s against the 2.5 PFLOP/s bf16 dense MFMA peak).
--workload ve times the training-side value-embedding gate forward and backward (nc_ve_forward, nc_ve_backward) at
the reference's d24 shape (GB/s of algorithmic bytes against 8 TB/s).
--workload fa times the training attention forward and backward (nc_flash_attn_fwd / _bwd) at the reference's d24
training shape (32 causal segments of 2048 tokens, 6 heads; TFLOP/s against the 2.5 PFLOP/s bf16 dense peak).
--workload c5 runs the end-to-end decoder (libnanochat_decode.so through the dec_* ABI): a random-init 26-layer
d1664 model, 128 random 2048-token prompts prefilled, then 512 greedy steps; value = decode tokens/s.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode-attn HBM GB/s (% of peak) + decode tokens/sec, bs64 ctx8K"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
PROFILES = ROOT / "profiles"


def attention_bytes(ctx_lens, q_heads, kv_heads):
    """Algorithmic bytes of one decode-attention launch: sum over (sequence, KV head)."""
    G = q_heads // kv_heads
    total = 0
    for n in ctx_lens:
        keys = int(n) + 1
        total += kv_heads * (keys * 264 + G * 128 * 2 * 2 + ((keys + 15) // 16) * 4)
    return total


def append_bytes(batch, kv_heads):
    """What the step's append adds to the attention's bytes: each token's k and v rows read, codes and scales
    written."""
    return batch * (2 * kv_heads * 256 + kv_heads * 264)


def traffic_from_profiles(kernel, workload):
    """HBM bytes per launch from the committed rocprofv3 counter summary, if one exists for this workload."""
    f = PROFILES / f"{kernel}_{workload}_traffic.json"
    if not f.exists():
        return None
    d = json.loads(f.read_text())
    return d.get("bytes_per_launch")


def cpu_baseline(w, inp, step_bytes, runs=5):
    """The CPU baseline of a decode workload: the PyTorch float32 restatement of the whole step (oracle/cpu_step.py:
    the step token's QK-norm/RoPE, fp8 quantize and store, gather + dequantize + attention) of every sequence, at
    every host thread, median of `runs` after one warm-up; the cache of the cached tokens is built untimed."""
    import torch

    from oracle import cpu_step as cs

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    B, Hq, Hkv = w.batch, w.q_heads, w.kv_heads
    table = inp["block_table"]
    ctx = inp["ctx_lens"].to(torch.int64)
    cache = cs.PagedCpuCache(inp["num_pages"], Hkv)
    for b in range(B):
        n = int(ctx[b])
        cache.store(table, b, torch.arange(n), inp["k_cache"][b, :n].float(), inp["v_cache"][b, :n].float())
    qkv = torch.cat([inp["q"].reshape(B, 1, -1), inp["k_new"].reshape(B, 1, -1), inp["v_new"].reshape(B, 1, -1)],
                    dim=2).float()
    ones = torch.ones(128)
    cos, sin = (torch.tensor(t) for t in _rotary(w.ctx + 2, 1e6))
    dt = cs.time_median(lambda: cs.step(cache, table, qkv, ctx, Hq, Hkv, ones, ones, cos, sin), runs=runs)
    return {"value": round(step_bytes / dt / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "cpu": cs.cpu_model(), "seconds_per_step": round(dt, 5),
            "sample": f"the whole step ({B} sequences, {int(ctx.sum()) + B} keys): PyTorch float32 restatement "
                      f"(oracle/cpu_step.py), torch.set_num_threads({threads}), median of {runs} after 1 warm-up"}


def _rotary(n, theta):
    from oracle.rope import rotary_tables

    return rotary_tables(n, theta)


def prefill_cpu_baseline(w, inp, flops, runs=5):
    """The CPU baseline of chunked prefill: the PyTorch float32 restatement of the step (the chunk's QK-norm/RoPE,
    quantize and store, then causal attention of every chunk row) at every host thread, median of `runs`."""
    import torch

    from oracle import cpu_step as cs

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    table, start = inp["block_table"], inp["start_pos"].to(torch.int64)
    cache = cs.PagedCpuCache(inp["num_pages"], w.kv_heads)
    for b in range(w.batch):
        cache.store(table, b, torch.arange(w.ctx), inp["k_cache"][b].float(), inp["v_cache"][b].float())
    cos, sin = (torch.tensor(t) for t in _rotary(w.ctx + w.chunk, w.theta))
    qkv = inp["qkv"].float()
    dt = cs.time_median(lambda: cs.step(cache, table, qkv, start, w.q_heads, w.kv_heads, inp["q_gain"],
                                        inp["k_gain"], cos, sin), runs=runs)
    return {"value": round(flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "cpu": cs.cpu_model(), "seconds_per_step": round(dt, 4),
            "sample": f"the whole step ({w.batch} x {w.chunk} rows onto {w.ctx}): PyTorch float32 restatement "
                      f"(oracle/cpu_step.py), torch.set_num_threads({threads}), median of {runs} after 1 warm-up"}


def prefill_flops(ctx, chunk, batch, q_heads):
    """Causal-useful FLOPs of chunked prefill: 4 * D per (query row, visible key), rows at ctx + i see ctx + i + 1."""
    keys = sum(ctx + i + 1 for i in range(chunk))
    return 4 * 128 * keys * batch * q_heads


def bench_prefill(args, w):
    """One chunked-prefill step of workload w (fused QK-norm/RoPE fp8 append of the chunk, then MFMA attention)."""
    import torch

    from nanochat_amd.attention import prefill_attention, qk_norm_rope_append
    from nanochat_amd.kv_cache import PagedKVCache
    from nanochat_amd.rotary import rotary_tables
    from nanochat_amd.workloads import prefill_inputs

    dev = torch.device("cuda:0")
    inp = prefill_inputs(w, seed=0)
    cache = PagedKVCache(inp["num_pages"], w.kv_heads, dev)
    table, start = inp["block_table"].to(dev), inp["start_pos"].to(dev)
    cache.append(inp["k_cache"].to(dev), inp["v_cache"].to(dev), torch.zeros_like(start), table, num_new=start)
    qkv = inp["qkv"].to(dev)
    qg, kg = inp["q_gain"].to(dev), inp["k_gain"].to(dev)
    cos, sin = rotary_tables(w.ctx + w.chunk, w.theta, dev)
    q = torch.empty(w.batch, w.chunk, w.q_heads, 128, dtype=torch.bfloat16, device=dev)
    out = torch.empty_like(q)

    def append():
        qk_norm_rope_append(qkv, w.q_heads, cache, table, start, qg, kg, cos, sin, q_out=q)

    def attend():
        prefill_attention(q, cache, table, start, out=out)

    for _ in range(args.warmup):
        append()
        attend()
    torch.cuda.synchronize()
    start_ev, stop_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start_ev.record()
    for _ in range(args.steps):
        append()
        attend()
    stop_ev.record()
    torch.cuda.synchronize()
    ms_step = start_ev.elapsed_time(stop_ev) / args.steps
    # the attention kernel's own duration: K back-to-back launches between two events on the launch stream (each
    # re-reads the same cache and writes the same rows), so no per-launch event sits between them
    start_ev.record()
    for _ in range(args.steps):
        attend()
    stop_ev.record()
    torch.cuda.synchronize()
    attn_ms = start_ev.elapsed_time(stop_ev) / args.steps
    flops = prefill_flops(w.ctx, w.chunk, w.batch, w.q_heads)
    achieved = flops / (attn_ms * 1e-3) / 1e12
    result = {
        "metric": "chunked-prefill attention TFLOP/s over the fp8 cache (MFMA)", "value": round(achieved, 2),
        "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp8e4m3 KV, fp8 QK^T and bf16 PV MFMA, fp32 softmax",
        "data": "synthetic (seeded N(0,1) bf16 chunk and cache, random-permutation block table)",
        "config": {"workload": f"{w.name}: {w.description}", "batch": w.batch, "q_heads": w.q_heads,
                   "kv_heads": w.kv_heads, "cached": w.ctx, "chunk": w.chunk, "rope_theta": w.theta},
        "attn_ms_mean": round(attn_ms, 5), "flops_per_launch": flops,
        "tokens_per_s": round(w.batch * w.chunk / (ms_step * 1e-3), 1),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "nc_prefill_attn_fp8 (prefill_lds_kernel)",
                     "timing": "HIP events around K back-to-back launches of the kernel on its stream"},
    }
    if args.cpu_seqs > 0:
        cpu = prefill_cpu_baseline(w, inp, flops)
        cpu["speedup_of_gpu_step"] = round(cpu["seconds_per_step"] / (ms_step * 1e-3), 1)
        result["cpu_baseline"] = cpu
    return result


VE_SHAPE = {"rows": 65536, "heads": 6, "vocab": 65536}   # reference d24 (C = 768), 32 x 2048 tokens


def ve_bytes(rows, heads, distinct):
    """Algorithmic HBM bytes of the value-embedding gate: forward reads n, v, idx and each distinct table row once,
    writes out and gate; backward reads dout, gate, ids, order and each distinct table row, writes dn and dz, and
    reads and writes each distinct dtable row."""
    C = heads * 128
    fwd = rows * (2 * C + 2 * C + 4 + 2 * C + 4 * heads) + distinct * 4 * C
    bwd = rows * (2 * C + 4 * heads + 4 + 8 + 2 * C + 2 * heads) + distinct * (4 * C + 8 * C)
    return fwd, bwd


def bench_ve(args):
    """The training-side value-embedding gate (nc_ve_forward, nc_ve_backward) at the reference's d24 shape."""
    import numpy as np
    import torch

    from nanochat_amd.native import check, hip_library, pointer, stream

    dev = torch.device("cuda:0")
    rows, H, V = VE_SHAPE["rows"], VE_SHAPE["heads"], VE_SHAPE["vocab"]
    C = H * 128
    gen = torch.Generator().manual_seed(0)
    qkv = torch.randn(rows, 3 * C, generator=gen).bfloat16().to(dev)
    n = torch.randn(rows, C, generator=gen).bfloat16().to(dev)
    table = torch.randn(V, C, generator=gen).to(dev)
    w = (torch.randn(H, C, generator=gen) * 0.05).to(dev)
    idx = torch.randint(0, V, (rows,), generator=gen, dtype=torch.int32)
    distinct = int(torch.unique(idx).numel())
    ids, order = torch.sort(idx.to(torch.int64), stable=True)
    idx, ids, order = idx.to(dev), ids.to(torch.int32).to(dev), order.to(dev)
    dqkv = torch.randn(rows, 3 * C, generator=gen).bfloat16().to(dev)
    out = torch.empty(rows, C, dtype=torch.bfloat16, device=dev)
    gate = torch.empty(rows, H, dtype=torch.float32, device=dev)
    dn, dz = torch.empty_like(out), torch.empty(rows, H, dtype=torch.bfloat16, device=dev)
    dtable = torch.zeros_like(table)
    lib = hip_library()
    v, dout = qkv[:, 2 * C:], dqkv[:, 2 * C:]

    def fwd():
        check(lib.nc_ve_forward(pointer(n), pointer(v), qkv.stride(0), pointer(idx), pointer(table), V, pointer(w),
                                pointer(out), pointer(gate), rows, H, stream()))

    def bwd():
        check(lib.nc_ve_backward(pointer(dout), dqkv.stride(0), pointer(ids), pointer(order), pointer(table), V,
                                 pointer(w), pointer(gate), pointer(dn), pointer(dtable), pointer(dz), rows, H,
                                 stream()))

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
        for a, b in evs:
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        return sorted(a.elapsed_time(b) for a, b in evs)

    f_ms, b_ms = timed(fwd), timed(bwd)
    fb, bb = ve_bytes(rows, H, distinct)
    f_med, b_med = f_ms[len(f_ms) // 2], b_ms[len(b_ms) // 2]
    f_gbs, b_gbs = fb / (f_med * 1e-3) / 1e9, bb / (b_med * 1e-3) / 1e9
    total = (fb + bb) / ((f_med + b_med) * 1e-3) / 1e9
    result = {
        "metric": "value-embedding gate forward + backward HBM GB/s", "value": round(total, 2), "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(f_med + b_med, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 activations, fp32 table/gate weights, fp32 accumulation",
        "data": "synthetic (seeded N(0,1) bf16 rows, uniform random tokens)",
        "config": {"workload": f"ve: {rows} rows (32 x 2048 tokens), H = {H} (C = {C}), vocab {V}, "
                               f"{distinct} distinct tokens", "rows": rows, "heads": H, "vocab": V},
        "forward": {"ms_median": round(f_med, 5), "bytes": fb, "gbs": round(f_gbs, 1),
                    "frac": round(f_gbs / HBM_PEAK_GBS, 4)},
        "backward": {"ms_median": round(b_med, 5), "bytes": bb, "gbs": round(b_gbs, 1),
                     "frac": round(b_gbs / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(total, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(total / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "ve_forward_kernel<6> + ve_backward_kernel<6>"},
    }
    if args.cpu_seqs > 0:
        result["cpu_baseline"] = ve_cpu_baseline(qkv, n, table, w, idx, dqkv, rows=rows)
    return result


def ve_cpu_baseline(qkv, n, table, w, idx, dqkv, rows):
    """The oracle (numpy, float64 sums) on the first `rows` rows of the same inputs: forward and backward."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import ve_gate as ov

    cores = min(16, os.cpu_count() or 1)
    H, C = w.shape[0], w.shape[1]
    nn = n[:rows].float().cpu().numpy()
    vv = qkv[:rows, 2 * C:].float().cpu().numpy()
    dd = dqkv[:rows, 2 * C:].float().cpu().numpy()
    tab, ww = table.cpu().numpy(), w.cpu().numpy()
    ii = idx[:rows].cpu().numpy().astype(np.int64)
    order = np.argsort(ii, kind="stable")
    with threadpool_limits(limits=cores):
        t0 = time.perf_counter()
        _, g = ov.ve_forward(nn, vv, ii, tab, ww)
        ov.ve_backward(dd, ii[order], order, tab, ww, g.astype(np.float32))
        dt = time.perf_counter() - t0
    fb, bb = ve_bytes(rows, H, len(np.unique(ii)))
    return {"value": round((fb + bb) / dt / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"oracle forward + backward (numpy) of the first {rows} of the rows, {dt:.2f} s"}


FA_SHAPE = {"segments": 32, "seqlen": 2048, "heads": 6}   # reference d24 training: 32 x 2048 tokens, C = 768


def fa_flops(segments, seqlen, heads, window=-1):
    """Causal-useful FLOPs of one forward: 4 * 128 per (row, visible key); the backward's algorithmic count is 2.5x
    (five products against the forward's two)."""
    keys = sum(min(i, window) + 1 if window >= 0 else i + 1 for i in range(seqlen))
    return 4 * 128 * keys * segments * heads


def bench_fa(args):
    """The training attention forward and backward (nc_flash_attn_fwd / _bwd) at the reference's d24 shape."""
    import torch

    from nanochat_amd.flash_attn import flash_attn_bwd, flash_attn_bwd_rows, flash_attn_fwd

    dev = torch.device("cuda:0")
    S, T, H = FA_SHAPE["segments"], FA_SHAPE["seqlen"], FA_SHAPE["heads"]
    gen = torch.Generator().manual_seed(0)
    q, k, v, do = (torch.randn(S * T, H, 128, generator=gen).bfloat16().to(dev) for _ in range(4))
    cu = torch.arange(0, S * T + 1, T, dtype=torch.int32, device=dev)
    out, lse = flash_attn_fwd(q, k, v, cu, T)
    rows = flash_attn_bwd_rows(out, do)

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
        for a, b in evs:
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        return sorted(a.elapsed_time(b) for a, b in evs)

    f_ms = timed(lambda: flash_attn_fwd(q, k, v, cu, T))
    b_ms = timed(lambda: flash_attn_bwd(q, k, v, out, do, lse, cu, T, rows=rows))
    f_med, b_med = f_ms[len(f_ms) // 2], b_ms[len(b_ms) // 2]
    ff = fa_flops(S, T, H)
    f_tf, b_tf = ff / (f_med * 1e-3) / 1e12, 2.5 * ff / (b_med * 1e-3) / 1e12
    total = 3.5 * ff / ((f_med + b_med) * 1e-3) / 1e12
    return {
        "metric": "training attention forward + backward TFLOP/s (causal, MFMA)", "value": round(total, 2),
        "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(f_med + b_med, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 MFMA, fp32 softmax and accumulation", "data": "synthetic (seeded N(0,1) bf16 q, k, v, dout)",
        "config": {"workload": f"fa: {S} segments x {T} tokens, {H} heads of 128, causal", "segments": S, "seqlen": T,
                   "heads": H},
        "forward": {"ms_median": round(f_med, 5), "flops": ff, "tflops": round(f_tf, 1),
                    "frac": round(f_tf / MFMA_BF16_PEAK_TFLOPS, 4)},
        "backward": {"ms_median": round(b_med, 5), "flops": int(2.5 * ff), "tflops": round(b_tf, 1),
                     "frac": round(b_tf / MFMA_BF16_PEAK_TFLOPS, 4),
                     "note": "algorithmic 2.5x forward; the two-kernel backward computes 3.5x"},
        "roofline": {"bound": "mfma", "achieved": round(total, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(total / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "flash_fwd_kernel + flash_bwd_dkv_kernel + flash_bwd_dq_kernel"},
    }


def model_decode_bytes(w, positions):
    """HBM bytes a decode step must read: every slot's cached keys (264 B per key per head per layer, positions
    0..p), the GEMM weights and lm_head in bf16."""
    H = w.hidden // 128
    kv = sum(p + 1 for p in positions) * w.layers * H * 264
    weights = 2 * (w.layers * (4 * w.hidden * w.hidden + 2 * w.hidden * w.ffn) + w.vocab * w.hidden)
    return kv + weights


def model_cpu_baseline(w, model, slots=16, steps=64, seed=0):
    """The CPU baseline of config 5: the PyTorch float32 restatement of the whole step (oracle/cpu_model.py, pinned
    against the float64 oracle) at every host thread, on a bounded sample: `steps` greedy decode steps of `slots`
    slots from the prompt's full context, over caches filled with seeded values (the step's work does not depend on
    them); tokens/s = slots * steps / time."""
    import torch

    from oracle.cpu_model import CpuDecoder
    from oracle.cpu_step import cpu_model

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    n = w.prompt - 1
    dec = CpuDecoder(model, slots, n + steps + 1, keep_codes=False)
    gen = torch.Generator().manual_seed(seed)
    for cache in (dec.k, dec.v):        # every cached element touched before the timed steps
        cache[:, :, :n].normal_(generator=gen)
    tokens = torch.randint(1, w.vocab, (slots,), generator=gen)
    dec.head(dec.body(tokens[:1], [n], [0]))   # warm-up (the step then rewrites position n)
    t0 = time.perf_counter()
    for s in range(steps):
        tokens = dec.head(dec.body(tokens, [n + s] * slots, list(range(slots)))).argmax(dim=-1)
    dt = time.perf_counter() - t0
    return {"value": round(slots * steps / dt, 3), "unit": "decode tokens/s", "cores": threads, "kind": "port",
            "cpu": cpu_model(),
            "sample": f"{steps} greedy decode steps of {slots} slots from context {n + 1} (caches pre-filled), "
                      f"PyTorch float32 restatement (oracle/cpu_model.py), torch.set_num_threads({threads})",
            "seconds": round(dt, 3)}


def bench_model(args, w, cpu_slots=16):
    """Config 5 end to end through the decoder runtime."""
    import torch

    from nanochat_amd.decoder import DecoderRuntime
    from nanochat_amd.workloads import model_tensors, prompt_tokens

    dev = torch.device("cuda:0")
    model = model_tensors(w.layers, w.hidden, w.ffn, w.vocab, w.max_length, seed=0, std=w.std, theta=w.theta,
                          softcap=w.softcap, device=dev, generator_device="cuda")
    ids = prompt_tokens(w.batch, w.prompt, w.vocab, seed=0).tolist()
    dec = DecoderRuntime(model, bos_token_id=0, max_length=w.max_length, prompt_store=0, max_slots=w.batch)
    try:
        if dec.batch < w.batch:
            raise RuntimeError(f"only {dec.batch} slots fit, the workload needs {w.batch}")
        # warm-up: a short prompt per slot and a few steps (the GEMM libraries load their kernels on first use)
        for b in range(w.batch):
            dec.place(b, ids[b][:32])
        dec.prefill()
        dec.activate(range(w.batch))
        for _ in range(max(1, min(args.warmup, 5))):
            dec.step()
        torch.cuda.synchronize()
        # prefill: every prompt but its last token (the first step's input), dec_prefill_rows rows a call
        t0 = time.perf_counter()
        for b in range(w.batch):
            dec.place(b, ids[b])
        dec.prefill()
        dec.stream.synchronize()
        prefill_s = time.perf_counter() - t0
        # decode: `steps` greedy steps of every slot, each ending with the tokens on the host (dec_tokens)
        positions = [w.prompt - 1] * w.batch
        step_bytes = 0
        t0 = time.perf_counter()
        for i in range(w.steps):
            dec.step()
            step_bytes += model_decode_bytes(w, [p + i for p in positions])
        decode_s = time.perf_counter() - t0
    finally:
        dec.close()
    tokens = w.batch * w.steps
    tok_s = tokens / decode_s
    roof_tok_s = tokens / (step_bytes / (HBM_PEAK_GBS * 1e9))
    prefill_rows = w.batch * (w.prompt - 1)
    H = w.hidden // 128
    prefill_flops_ = 2 * prefill_rows * (w.layers * (4 * w.hidden * w.hidden + 2 * w.hidden * w.ffn)) + \
        4 * 128 * H * w.batch * (w.layers - 1) * sum(range(1, w.prompt))
    result = {
        "metric": "end-to-end decode tokens/s (config 5)", "value": round(tok_s, 1), "unit": "tokens/s",
        "n_gpus": 1, "steps": w.steps, "warmup": args.warmup, "ms_per_step": round(1e3 * decode_s / w.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 weights/activations, fp8e4m3 KV, fp32 accumulation",
        "data": "synthetic (random-init N(0, 0.02) weights, random-token prompts, seeded)",
        "config": {"workload": f"{w.name}: {w.description}", "layers": w.layers, "hidden": w.hidden,
                   "heads": H, "ffn": w.ffn, "vocab": w.vocab, "batch": w.batch, "prompt": w.prompt,
                   "steps": w.steps, "rope_theta": w.theta},
        "prefill_s": round(prefill_s, 4), "prefill_tokens_per_s": round(prefill_rows / prefill_s, 1),
        "prefill_tflops": round(prefill_flops_ / prefill_s / 1e12, 2),
        "decode_s": round(decode_s, 4), "end_to_end_tokens_per_s": round(tokens / (prefill_s + decode_s), 1),
        "roofline": {"bound": "hbm", "achieved": round(step_bytes / decode_s / 1e9, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(tok_s / roof_tok_s, 4), "traffic": None,
                     "kernel": "whole decode step (KV + weights per step)",
                     "roofline_tokens_per_s": round(roof_tok_s, 1)},
    }
    if cpu_slots > 0:
        result["cpu_baseline"] = model_cpu_baseline(w, model, cpu_slots)
        result["cpu_baseline"]["speedup_of_gpu"] = round(tok_s / result["cpu_baseline"]["value"], 1)
    return result


def bench_ceiling(args):
    """The read-only ceiling of a decode workload's step: its algorithmic bytes (attention and append) read as
    2 KiB pages by nc_debug_read_pages, in page order and in a seeded random order (the block table's kind), at
    two grid sizes; args.steps launches timed between events on the launch stream after args.warmup."""
    import torch

    from nanochat_amd import native
    from nanochat_amd.workloads import DECODE, decode_ctx_lens

    w = DECODE[args.workload]
    ctx = decode_ctx_lens(w, torch.Generator().manual_seed(0))
    step_bytes = attention_bytes(ctx.tolist(), w.q_heads, w.kv_heads) + append_bytes(w.batch, w.kv_heads)
    pages = step_bytes // 2048
    dev = torch.device("cuda:0")
    src = torch.randint(0, 256, (pages * 2048,), dtype=torch.uint8, device=dev)
    orders = {"page order": None,
              "random order": torch.randperm(pages, generator=torch.Generator().manual_seed(1)).to(torch.int32).to(dev)}
    lib = native.hip_library()
    rows = []
    for name, order in orders.items():
        for grid in (1024, 2048):
            sink = torch.empty(grid * 256, dtype=torch.int32, device=dev)

            def launch():
                rc = lib.nc_debug_read_pages(native.pointer(src), src.numel(), native.pointer(order) if order is not None
                                             else None, pages, grid, native.pointer(sink), native.stream())
                if rc:
                    raise RuntimeError(f"nc_debug_read_pages: {lib.nc_status_string(rc).decode()}")

            for _ in range(args.warmup):
                launch()
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            start.record()
            for _ in range(args.steps):
                launch()
            stop.record()
            torch.cuda.synchronize()
            us = start.elapsed_time(stop) * 1e3 / args.steps
            rows.append({"order": name, "grid": grid, "us": round(us, 2),
                         "tb_per_s": round(pages * 2048 / us / 1e6, 3)})
    best = max(r["tb_per_s"] for r in rows if r["order"] == "random order")
    return {"metric": "read-only HBM ceiling of the decode step's bytes", "value": best, "unit": "TB/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
            "data": "synthetic (random bytes)", "frac_of_8tbs": round(best / 8.0, 4),
            "config": {"workload": args.workload, "bytes": pages * 2048, "pages": pages,
                       "kernel": "read_pages_kernel (nc_debug_read_pages)"}, "runs": rows}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c3u")
    ap.add_argument("--workers", type=int, default=0, help="decode: waves taking the work items (0: all slots)")
    ap.add_argument("--cpu-seqs", type=int, default=64,
                    help="CPU baseline: 0 skips it; decode and prefill time the whole step, c5 this many slots (<= 16)")
    ap.add_argument("--two-launch", action="store_true",
                    help="decode: the step as nc_qk_norm_rope_append_fp8 + nc_decode_attn_fp8 (the same bits)")
    ap.add_argument("--ceiling", action="store_true",
                    help="decode workloads: time a read-only pass over the step's bytes (the memory system's ceiling)")
    ap.add_argument("--no-e2e", action="store_true",
                    help="decode workloads: skip the config-5 end-to-end decode tokens/s part of the metric")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: the fp8 KV decode path is single-GPU by design (asked for {args.gpus})",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from nanochat_amd.attention import decode_attention, decode_step, decode_workspace_bytes, qk_norm_rope_append
    from nanochat_amd.kv_cache import PagedKVCache
    from nanochat_amd.rotary import rotary_tables
    from nanochat_amd.workloads import DECODE, decode_inputs

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    from nanochat_amd.workloads import MODELS, PREFILL

    if args.workload == "ve":
        print(json.dumps(bench_ve(args)), flush=True)
        return
    if args.workload == "fa":
        print(json.dumps(bench_fa(args)), flush=True)
        return
    if args.workload in PREFILL:
        print(json.dumps(bench_prefill(args, PREFILL[args.workload])), flush=True)
        return
    if args.ceiling:
        print(json.dumps(bench_ceiling(args)), flush=True)
        return
    if args.workload in MODELS:
        print(json.dumps(bench_model(args, MODELS[args.workload], cpu_slots=min(args.cpu_seqs, 16))), flush=True)
        return
    dev = torch.device("cuda:0")
    w = DECODE[args.workload]
    inp = decode_inputs(w, seed=0)
    B, Hq, Hkv = w.batch, w.q_heads, w.kv_heads

    # resident state: the cache (built through the append entry point), the step's inputs and outputs
    cache = PagedKVCache(inp["num_pages"], Hkv, dev)
    table = inp["block_table"].to(dev)
    ctx = inp["ctx_lens"].to(dev)
    cache.append(inp["k_cache"].to(dev), inp["v_cache"].to(dev), torch.zeros_like(ctx), table, num_new=ctx)
    qkv = torch.cat([inp["q"].reshape(B, 1, -1), inp["k_new"].reshape(B, 1, -1), inp["v_new"].reshape(B, 1, -1)],
                    dim=2).contiguous().to(dev)
    gain = torch.ones(128, dtype=torch.float32, device=dev)
    cos, sin = rotary_tables(w.ctx + 2, 1e6, dev)
    seq_lens = ctx + 1
    q_out = torch.empty(B, 1, Hq, 128, dtype=torch.bfloat16, device=dev)
    out = torch.empty(B, Hq, 128, dtype=torch.bfloat16, device=dev)
    ws = torch.zeros(max(1, decode_workspace_bytes(B, Hq, Hkv, inp["max_seq_len"], -1)),
                     dtype=torch.uint8, device=dev)

    if args.two_launch:
        def step():
            qk_norm_rope_append(qkv, Hq, cache, table, ctx, gain, gain, cos, sin, q_out=q_out)
            decode_attention(q_out.view(B, Hq, 128), cache, table, seq_lens, inp["max_seq_len"],
                             workers=args.workers, out=out, workspace=ws)
    else:
        qkv_rows = qkv.view(B, -1)

        def step():
            decode_step(qkv_rows, Hq, cache, table, seq_lens, gain, gain, cos, sin, inp["max_seq_len"],
                        workers=args.workers, out=out, workspace=ws)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # timed region: K whole steps between two events on the launch stream
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        step()
    stop.record()
    torch.cuda.synchronize()
    ms_step = start.elapsed_time(stop) / args.steps

    # the spread of single launches, each between its own pair of events (an event pair adds a few microseconds; the
    # roofline uses the back-to-back mean above)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for a, b in evs:
        a.record()
        step()
        b.record()
    torch.cuda.synchronize()
    attn_ms = sorted(a.elapsed_time(b) for a, b in evs)
    attn_mean_ms = sum(attn_ms) / len(attn_ms)

    attn_b = attention_bytes(inp["ctx_lens"].tolist(), Hq, Hkv)
    step_b = attn_b + append_bytes(B, Hkv)
    value = step_b / (ms_step * 1e-3) / 1e9
    achieved = step_b / (ms_step * 1e-3) / 1e9
    traffic = traffic_from_profiles("decode_step", args.workload)
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3 KV, fp8 QK^T and bf16 PV MFMA, fp32 softmax",
        "data": "synthetic (seeded N(0,1) bf16, 1% 8-sigma outliers, random-permutation block table)",
        "config": {"workload": f"{w.name}: {w.description}", "batch": B, "q_heads": Hq, "kv_heads": Hkv,
                   "keys_per_seq": inp["max_seq_len"], "page_size": 16,
                   "step": ("QK-norm/RoPE fp8 append, then split-K decode attention (two launches)" if args.two_launch
                            else "fused decode step: QK-norm/RoPE fp8 append + split-K decode attention, one launch"),
                   "workers": args.workers or "auto"},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "decode_tokens_per_s_per_layer": round(B / (ms_step * 1e-3), 1),
        "event_bracketed_launch_ms_mean": round(attn_mean_ms, 5),
        "event_bracketed_launch_ms_p10_p50_p90": [round(attn_ms[len(attn_ms) // 10], 5), round(attn_ms[len(attn_ms) // 2], 5),
                                  round(attn_ms[9 * len(attn_ms) // 10], 5)],
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": ("qk_norm_rope append_kernel + decode_kernel<false>" if args.two_launch
                                else "nc_decode_step_fp8 (decode_kernel<true, false>)"),
                     "bytes_per_launch": step_b,
                     "timing": "HIP events around K back-to-back launches of the kernel on its stream"},
    }
    if args.cpu_seqs > 0:
        result["cpu_baseline"] = cpu_baseline(w, inp, step_b)
        result["cpu_baseline"]["speedup_of_gpu_step"] = round(value / result["cpu_baseline"]["value"], 1)
    if not args.no_e2e:
        # the metric's second half: end-to-end decode tokens/s of config 5 through the decoder runtime
        del cache, ws, qkv, q_out, out
        torch.cuda.empty_cache()
        e2e = bench_model(args, MODELS["c5"], cpu_slots=16 if args.cpu_seqs > 0 else 0)
        result["decode_tokens_per_s"] = e2e["value"]
        keep = ("metric", "value", "unit", "ms_per_step", "config", "prefill_s", "prefill_tokens_per_s",
                "prefill_tflops", "decode_s", "end_to_end_tokens_per_s", "roofline", "cpu_baseline")
        result["end_to_end"] = {k: e2e[k] for k in keep if k in e2e}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
