"""Benchmark: paged 4-bit KV decode attention + KV append (config 3).

Workload ("Paged continuous batching", the configuration the headline metric is
quoted on): a pool of
16384 blocks x 32 tokens per layer, bf16 inputs stored affine 4-bit g64,
8 KV heads x 128 dims; 64 sequences with lengths U[128, 8192] whose block
tables are random permutations of pool ids; 32 sequences share one
refcounted 2048-token prefix (64 blocks).  One step = for each of the
--layers layers: append one token per sequence plus one 512-token
chunked-prefill chunk (one append call for the step's 576 new tokens), then
decode attention (32 query heads) over every sequence.  Synthetic data, generated on the GPU; all inputs are resident in
HBM before timing starts.  The step writes the decode token at the same
position each step, so every step does identical work.

Prints one JSON line: "value" is the whole-step KV-read rate (appends included),
"attention" times the paged decode call (one launch: the decode kernel
merges its split-K partials itself), "roofline" that decode launch (the
library's event pair around it, on its launch stream), "traffic" is the PMC-measured HBM bytes per decode launch,
"cpu_baseline" times the C oracle, "prefill" times a 512-token chunked-prefill
attention step over a 4-bit cache, and "mla" is the MLA latent decode workload
(32 x 16384 tokens, 128 heads) with the MFMA roofline of its attention kernel.
"configs" measures the other benchmark workloads at their stated shapes, each
with the roofline of its decode kernel: config 1 (KVCacheSimple fp16 decode
steps), config 2 (QuantizedKVCache, 32 layers x batch 8 x 4096 tokens, 4 and
8 bits) and config 4 (5 sliding-window + 1 global 8-bit layer at 32768).
`--only <leg>` runs one workload alone (for profiling).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "vmlx-swift_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
BYTES_PER_TOKEN_HEAD = 144  # 4-bit K+V codes (2 x 64 B) + 2 groups x (scale+bias) x 2 B x 2


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=32)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-threads", type=int, default=0)
    p.add_argument("--no-mla", action="store_true",
                   help="skip the MLA latent decode measurement (config 5)")
    p.add_argument("--only", default="all",
                   choices=["all", "config3", "config1", "config2", "config4", "mla", "prefill",
                            "turboquant"],
                   help="run one workload only (profiling); the JSON line needs 'all'")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="only run a plain 1 GiB device copy (vkv_array_copy) 5 times: the "
                        "reference reading for the FETCH_SIZE / WRITE_SIZE counters")
    return p.parse_args()


def pmc_traffic():
    """HBM bytes per decode launch from the committed PMC summary (two
    rocprofv3 --pmc passes, FETCH_SIZE and WRITE_SIZE, scaled by a 1 GiB copy
    calibration); None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "qdecode_config3_traffic.txt")
    if not os.path.exists(path):
        return None
    vals = {}
    for line in open(path):
        parts = line.split()
        if len(parts) == 2 and not line.startswith("#"):
            vals[parts[0]] = int(parts[1])
    if "read_bytes" not in vals or "write_bytes" not in vals:
        return None
    return vals["read_bytes"] + vals["write_bytes"]


def calibrate_copy(torch, vkv):
    n = 1 << 28  # f32 elements = 1 GiB read + 1 GiB written per launch
    a = torch.ones((1, 1, n // 64, 64), dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    for _ in range(5):
        vkv._chk(vkv.lib().vkv_array_copy(vkv.C.byref(vkv.arr(a)), vkv.C.byref(vkv.arr(b)),
                                          vkv.stream_ptr()))
    torch.cuda.synchronize()
    assert bool((b == 1).all())
    print(json.dumps({"calibrate_copy_bytes_per_launch": 4 * n, "launches": 5}), flush=True)


def build_scene(torch, vkv, layers, seed=3):
    import numpy as np

    rng = np.random.default_rng(seed)
    nblocks, bs, H, D, Hq = 16384, 32, 8, 128, 32
    n_seqs, share_tokens, n_share, prefill = 64, 2048, 32, 512
    lens = rng.integers(128, 8193, n_seqs)
    sharers = [i for i in range(n_seqs) if lens[i] > share_tokens][:n_share]
    perm = rng.permutation(np.arange(1, nblocks))
    nxt = 0

    def take(n):
        nonlocal nxt
        out = perm[nxt:nxt + n]
        nxt += n
        return list(out)

    shared = take(share_tokens // bs)
    tables = []
    for s in range(n_seqs):
        L = int(lens[s]) + 1  # + the decode token
        nb = (L + bs - 1) // bs
        if s in sharers:
            t = shared + take(nb - len(shared))
        else:
            t = take(nb)
        tables.append(t)
    prefill_blocks = take(prefill // bs)
    width = max(len(t) for t in tables)
    tab = np.zeros((n_seqs, width), np.int32)
    for s, t in enumerate(tables):
        tab[s, :len(t)] = t
    # slots: initial fill (each shared block written once), decode tokens, prefill chunk
    fill_slots = []
    for s in range(n_seqs):
        start = share_tokens if (s in sharers and s != sharers[0]) else 0
        fill_slots += [tables[s][p // bs] * bs + p % bs for p in range(start, int(lens[s]))]
    dec_slots = [tables[s][int(lens[s]) // bs] * bs + int(lens[s]) % bs for s in range(n_seqs)]
    pre_slots = [prefill_blocks[p // bs] * bs + p % bs for p in range(prefill)]
    dev = dict(device="cuda")
    sc = dict(
        nblocks=nblocks, bs=bs, H=H, D=D, Hq=Hq, n_seqs=n_seqs, lens=lens, sharers=sharers,
        share_tokens=share_tokens, prefill=prefill,
        table=torch.from_numpy(tab).to(**dev),
        seq_lens=torch.from_numpy((lens + 1).astype(np.int32)).to(**dev),
        max_len=int(lens.max()) + 1,
        fill_slots=torch.tensor(fill_slots, dtype=torch.int32, **dev),
        dec_slots=torch.tensor(dec_slots, dtype=torch.int32, **dev),
        pre_slots=torch.tensor(pre_slots, dtype=torch.int32, **dev),
    )
    pool = vkv.PagedPool(nblocks, bs, layers, H, D, dtype=vkv.BF16, bits=4)
    nfill = len(fill_slots)
    stage_k = torch.empty((nfill, H, D), dtype=torch.bfloat16, **dev)
    stage_v = torch.empty_like(stage_k)
    for l in range(layers):
        vkv.fill_normal(stage_k, seed=1000 + 2 * l)
        vkv.fill_normal(stage_v, seed=1001 + 2 * l)
        pool.append(l, stage_k, stage_v, sc["fill_slots"])
    del stage_k, stage_v
    sc["q"] = vkv.fill_normal(torch.empty((layers, n_seqs, Hq, D), dtype=torch.bfloat16, **dev), 7)
    sc["dk"] = vkv.fill_normal(torch.empty((layers, n_seqs, H, D), dtype=torch.bfloat16, **dev), 8)
    sc["dv"] = vkv.fill_normal(torch.empty((layers, n_seqs, H, D), dtype=torch.bfloat16, **dev), 9)
    sc["pk"] = vkv.fill_normal(torch.empty((layers, prefill, H, D), dtype=torch.bfloat16, **dev), 10)
    sc["pv"] = vkv.fill_normal(torch.empty((layers, prefill, H, D), dtype=torch.bfloat16, **dev), 11)
    # a step's new tokens (the decode token of every sequence, then the
    # prefill chunk) are appended with one call per layer, as a batching
    # engine issues them
    sc["ak"] = torch.cat([sc["dk"], sc["pk"]], dim=1).contiguous()
    sc["av"] = torch.cat([sc["dv"], sc["pv"]], dim=1).contiguous()
    sc["all_slots"] = torch.cat([sc["dec_slots"], sc["pre_slots"]]).contiguous()
    sc["out"] = torch.empty((layers, n_seqs, Hq, D), dtype=torch.bfloat16, **dev)
    sc["views"] = [pool.view(l, sc["table"], sc["seq_lens"], sc["max_len"]) for l in range(layers)]
    torch.cuda.synchronize()
    return pool, sc


def prefill_measure(torch, vkv, steps, warmup):
    """The chunked-prefill step of a config-3-shaped layer: a 512-token
    causal chunk appended to a 4-bit g64 QuantizedKVCache that holds a
    4096-token prefix (32 query / 8 kv heads x 128, bf16), then attention of
    the chunk over all 4608 tokens through attentionWithCacheUpdate.  One
    step = one call (append + page gather + multi-query kernel), timed with
    HIP events; the cache is trimmed back after each call."""
    Hq, Hkv, D, T0, L = 32, 8, 128, 4096, 512
    cache = vkv.QuantizedKVCache(group_size=64, bits=4)
    k0 = torch.empty((1, Hkv, T0, D), dtype=torch.bfloat16, device="cuda")
    v0 = torch.empty_like(k0)
    vkv.fill_normal(k0, seed=31)
    vkv.fill_normal(v0, seed=32)
    cache.update_quantized(k0, v0)
    q = torch.empty((1, Hq, L, D), dtype=torch.bfloat16, device="cuda")
    k1 = torch.empty((1, Hkv, L, D), dtype=torch.bfloat16, device="cuda")
    v1 = torch.empty_like(k1)
    for t, sd in ((q, 33), (k1, 34), (v1, 35)):
        vkv.fill_normal(t, seed=sd)
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream()

    def call():
        vkv.attention_with_cache_update(q, k1, v1, cache, D ** -0.5, mask="causal", out=out)
        cache.trim(L)

    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        call()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flops = 2.0 * 2 * Hq * D * L * (T0 + (L + 1) / 2)  # QK + PV over the causal keys
    return {"workload": "chunked prefill: 512-token causal chunk over a 4096-token 4-bit g64 "
                        "QuantizedKVCache, 32/8 heads x 128, bf16",
            "ms_per_chunk": round(ms, 5), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
            "finite": bool(torch.isfinite(out.float()).all())}


def mla_measure(torch, vkv, steps, warmup):
    """Config 5: MLA absorbed decode over an 8-bit g64 latent pool (576-dim
    entries, 64-token blocks), 32 sequences x 16384 tokens, 128 query heads.
    One step = one vkv_mla_decode call (main kernel + split combine), timed
    with HIP events on the launching stream."""
    B, T, H, DK, DV, BS = 32, 16384, 128, 576, 512, 64
    nb = B * T // BS + 1
    pool = vkv.PagedPool(nb, BS, 1, 1, DK, dtype=vkv.BF16, bits=8, group_size=64, v_head_dim=DV,
                         flags=vkv.VIEW_KEYS_ONLY)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    table = (torch.randperm(nb - 1, device="cuda", generator=gen).int() + 1).view(B, T // BS)
    table = table.contiguous()
    slots = (table.view(-1, 1) * BS + torch.arange(BS, device="cuda", dtype=torch.int32)).view(-1)
    chunk = 65536
    x = torch.empty((chunk, 1, DK), dtype=torch.bfloat16, device="cuda")
    for c in range(0, B * T, chunk):
        vkv.fill_normal(x, seed=17 + c, std=0.5)   # latent ~ N(0, 0.5)
        pool.append(0, x, None, slots[c:c + chunk].contiguous())
    lens = torch.full((B,), T, dtype=torch.int32, device="cuda")
    view = pool.view(0, table, lens, T)
    q = torch.empty((B, H, DK), dtype=torch.bfloat16, device="cuda")
    vkv.fill_normal(q, seed=23)
    out = torch.empty((B, H, DV), dtype=torch.bfloat16, device="cuda")
    scale = 192 ** -0.5
    stream = torch.cuda.current_stream()

    def call():
        vkv._chk(vkv.lib().vkv_mla_decode(
            vkv.C.byref(vkv.arr(q)), vkv.C.byref(view), vkv.C.c_float(scale),
            vkv.C.byref(vkv.arr(out)), vkv.stream_ptr()))

    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        call()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # the attention kernel alone (without the split merge), from the
    # library's event pair around it, over the same number of calls
    vkv.kernel_timing(True)
    for _ in range(steps):
        call()
    k_ms, k_n = vkv.kernel_timing_read(vkv.TIME_MLA)
    vkv.kernel_timing(False)
    k_ms /= max(k_n, 1)
    kv_bytes = B * T * (DK + (DK // 64) * 4)          # 612 B per entry
    flops = 2.0 * H * B * T * (DK + DV)
    tflops = flops / (ms * 1e-3) / 1e12
    k_tflops = flops / (k_ms * 1e-3) / 1e12
    del pool
    return {
        "workload": "MLA absorbed decode: 32 seqs x 16384 tokens, 576-dim latent+rope entries "
                    "8-bit g64 (9 groups) in 64-token pages, 128 query heads, out 512 dims",
        "ms_per_step": round(ms, 4),
        "kv_gbs": round(kv_bytes / (ms * 1e-3) / 1e9, 1),
        "tflops": round(tflops, 1),
        "kernel_ms": round(k_ms, 5),
        "roofline": {"bound": "mfma", "achieved": round(k_tflops, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(k_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                     "kernel": "mla_kernel"},
        "finite": bool(torch.isfinite(out.float()).all()),
    }


def _time_calls(torch, vkv, fn, steps, warmup, kind=None):
    """Milliseconds per call of fn (HIP events on the current stream around
    `steps` calls after `warmup`), and, when `kind` is given, the average
    duration and count of the library-timed kernel of that kind over a
    second set of `steps` calls."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    if kind is None:
        return ms, None, 0
    vkv.kernel_timing(True)
    for _ in range(steps):
        fn()
    k_ms, k_n = vkv.kernel_timing_read(kind)
    vkv.kernel_timing(False)
    return ms, k_ms / max(k_n, 1), k_n


def _roofline(byts, k_ms, kernel):
    gbs = byts / (k_ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "kernel": kernel,
            "kernel_us": round(k_ms * 1e3, 2), "bytes_per_launch": int(byts)}


def config1_measure(torch, vkv, steps, warmup):
    """Config 1: KVCacheSimple single layer, fp16, batch 1, 8 KV heads x 128:
    a 512-token prefill update, then 64 single-token decode steps, each an
    update plus decode attention (32 query heads) through
    attentionWithCacheUpdate.  One pass = the 64 decode steps; the cache is
    trimmed back to 512 tokens between passes (capacity stays 768)."""
    H, Hq, D, T0, N = 8, 32, 128, 512, 64
    f16 = dict(dtype=torch.float16, device="cuda")
    pk = vkv.fill_normal(torch.empty((1, H, T0, D), **f16), 41)
    pv = vkv.fill_normal(torch.empty((1, H, T0, D), **f16), 42)
    dk = vkv.fill_normal(torch.empty((N, 1, H, 1, D), **f16), 43)
    dv = vkv.fill_normal(torch.empty((N, 1, H, 1, D), **f16), 44)
    q = vkv.fill_normal(torch.empty((N, 1, Hq, 1, D), **f16), 45)
    out = torch.empty((1, Hq, 1, D), **f16)

    def prefill():
        c = vkv.KVCacheSimple()
        c.update(pk, pv)
        return c

    cache = prefill()

    def decode_pass():
        for i in range(N):
            vkv.attention_with_cache_update(q[i], dk[i], dv[i], cache, D ** -0.5, out=out)
        cache.trim(N)

    pass_ms, k_ms, k_n = _time_calls(torch, vkv, decode_pass, steps, warmup, vkv.TIME_FDECODE)
    pre_ms, _, _ = _time_calls(torch, vkv, prefill, steps, warmup)
    kv_bytes = sum((T0 + i + 1) * H * D * 2 * 2 for i in range(N))  # K + V read per pass
    step_ms = pass_ms / N
    return {
        "workload": "KVCacheSimple fp16, B1, 8/32 heads x 128: 512-token prefill update, then "
                    "64 decode steps (update + SDPA through attentionWithCacheUpdate)",
        "decode_step_us": round(step_ms * 1e3, 2),
        "decode_tokens_per_s": round(1e3 / step_ms, 1),
        "decode_kv_gbs": round(kv_bytes / (pass_ms * 1e-3) / 1e9, 1),
        "prefill_update_us": round(pre_ms * 1e3, 2),
        "roofline": _roofline(kv_bytes / N, k_ms, "fdecode_kernel"),
        "note": "2.1-2.4 MB per step: launch-latency bound, not bandwidth bound",
    }


def _outlier_scale(torch, B, H, D, gen):
    """[B, H, 1, D] multipliers: 20 on 4 random channels per (batch, head)."""
    m = torch.ones((B, H, 1, D), dtype=torch.bfloat16, device="cuda")
    ch = torch.rand((B, H, D), device="cuda", generator=gen).argsort(-1)[..., :4]
    m.view(B, H, D).scatter_(-1, ch, 20.0)
    return m


def config2_measure(torch, vkv, steps, warmup, bits, ref=0):
    """Config 2: QuantizedKVCache at Llama-3-8B layer shapes -- 32 layers,
    batch 8, 8 KV / 32 query heads x 128, a 4096-token context, bf16 K/V
    ~ N(0,1) with 4 channels per head x20, affine g64 at `bits`.  One step =
    for each layer, updateQuantized of one token and quantized decode
    attention through attentionWithCacheUpdate; each cache is trimmed back by
    the token after the step.  ref = 1: with the reference_softmax option
    (the reference's bf16 softmax in a pass of its own; the roofline then
    times the P.V pass)."""
    layers, B, H, Hq, D, T0 = 32, 8, 8, 32, 128, 4096
    gen = torch.Generator(device="cuda")
    gen.manual_seed(200 + bits)
    bf = dict(dtype=torch.bfloat16, device="cuda")
    caches = [vkv.QuantizedKVCache(group_size=64, bits=bits) for _ in range(layers)]
    stage = torch.empty((B, H, T0, D), **bf)
    stage2 = torch.empty_like(stage)
    for l, c in enumerate(caches):
        m = _outlier_scale(torch, B, H, D, gen)
        vkv.fill_normal(stage, 300 + 2 * l)
        vkv.fill_normal(stage2, 301 + 2 * l)
        c.update_quantized(stage * m, stage2 * m)
    del stage, stage2
    dk = vkv.fill_normal(torch.empty((layers, B, H, 1, D), **bf), 51)
    dv = vkv.fill_normal(torch.empty((layers, B, H, 1, D), **bf), 52)
    q = vkv.fill_normal(torch.empty((layers, B, Hq, 1, D), **bf), 53)
    out = torch.empty((layers, B, Hq, 1, D), **bf)

    def step():
        for l, c in enumerate(caches):
            vkv.attention_with_cache_update(q[l], dk[l], dv[l], c, D ** -0.5, out=out[l])
        for c in caches:
            c.trim(1)

    vkv.set_option("reference_softmax", ref)
    try:
        ms, k_ms, k_n = _time_calls(torch, vkv, step, steps, warmup, vkv.TIME_DECODE)
    finally:
        vkv.set_option("reference_softmax", 0)
    per_tok = 2 * (D * bits // 8 + (D // 64) * 4)          # K + V codes + scale/bias
    layer_bytes = B * H * (T0 + 1) * per_tok
    finite = bool(torch.isfinite(out.float()).all())
    del caches
    return {
        "workload": f"QuantizedKVCache {bits}-bit g64, 32 layers, B8, 8/32 heads x 128, "
                    f"context 4096 (+1 decode token), x20 outlier channels"
                    + (", reference softmax" if ref else ""),
        "ms_per_step": round(ms, 4),
        "step_kv_gbs": round(layers * layer_bytes / (ms * 1e-3) / 1e9, 1),
        "roofline": _roofline(layer_bytes, k_ms, "qdecode_kernel"),
        "finite": finite,
    }


def config4_measure(torch, vkv, steps, warmup):
    """Config 4: Gemma-style layers at 16 query / 8 KV heads x 256, batch 4,
    bf16 ~ N(0,1): 5 sliding-window layers (RotatingKVCache(maxSize: 1024),
    filled past a wrap so every decode writes in place into a full ring) and
    1 global layer (8-bit g64 QuantizedKVCache at a 32768-token context).
    One step = a decode token through attentionWithCacheUpdate on each of
    the 6 layers; the global cache is trimmed back after the step."""
    B, Hq, H, D, M, T0, n_win = 4, 16, 8, 256, 1024, 32768, 5
    bf = dict(dtype=torch.bfloat16, device="cuda")
    wins = [vkv.RotatingKVCache(M) for _ in range(n_win)]
    pre = torch.empty((B, H, M + 100, D), **bf)
    for l, c in enumerate(wins):
        vkv.fill_normal(pre, 400 + l)
        c.update(pre[:, :, :M - 1], pre[:, :, :M - 1])
        for t in range(M - 1, M + 100):          # fill the ring and wrap it
            c.update(pre[:, :, t:t + 1], pre[:, :, t:t + 1])
    del pre
    glob = vkv.QuantizedKVCache(group_size=64, bits=8)
    stage = vkv.fill_normal(torch.empty((B, H, T0 - 1, D), **bf), 410)
    glob.update_quantized(stage, vkv.fill_normal(stage.clone(), 411))
    del stage
    dk = vkv.fill_normal(torch.empty((n_win + 1, B, H, 1, D), **bf), 61)
    dv = vkv.fill_normal(torch.empty((n_win + 1, B, H, 1, D), **bf), 62)
    q = vkv.fill_normal(torch.empty((n_win + 1, B, Hq, 1, D), **bf), 63)
    out = torch.empty((n_win + 1, B, Hq, 1, D), **bf)
    scale = D ** -0.5

    def win_layers():
        for l, c in enumerate(wins):
            vkv.attention_with_cache_update(q[l], dk[l], dv[l], c, scale, out=out[l])

    def glob_layer():
        vkv.attention_with_cache_update(q[n_win], dk[n_win], dv[n_win], glob, scale, out=out[n_win])
        glob.trim(1)

    def step():
        win_layers()
        glob_layer()

    ms, _, _ = _time_calls(torch, vkv, step, steps, warmup)
    w_ms, wk_ms, _ = _time_calls(torch, vkv, win_layers, steps, warmup, vkv.TIME_FDECODE)
    g_ms, gk_ms, _ = _time_calls(torch, vkv, glob_layer, steps, warmup, vkv.TIME_DECODE)
    win_bytes = B * H * M * D * 2 * 2
    glob_bytes = B * H * T0 * 2 * (D + (D // 64) * 4)
    step_bytes = n_win * win_bytes + glob_bytes
    finite = bool(torch.isfinite(out.float()).all())
    return {
        "workload": "Gemma-style: 5 sliding-window layers (RotatingKVCache maxSize 1024, full "
                    "ring) + 1 global layer (8-bit g64, context 32768); B4, 16/8 heads x 256",
        "ms_per_step": round(ms, 4),
        "step_kv_gbs": round(step_bytes / (ms * 1e-3) / 1e9, 1),
        "window_layer_us": round(w_ms * 1e3 / n_win, 2),
        "window_layer_pct_hbm_peak": round(100 * win_bytes / (w_ms / n_win * 1e-3) / 1e9
                                           / HBM_PEAK_GBS, 2),
        "global_layer_us": round(g_ms * 1e3, 2),
        "roofline_window": _roofline(win_bytes, wk_ms, "fdecode_kernel"),
        "roofline_global": _roofline(glob_bytes, gk_ms, "qdecode_kernel"),
        "finite": finite,
    }


def cpu_baseline(threads, min_seconds=8.0):
    """The CPU oracle (C restatement of the reference arithmetic: scores and
    the softmax in bf16 as softmax(precise: false) computes them, fp64
    accumulation elsewhere) on one layer of the same workload: the 64
    config-3 sequences (same lengths as the GPU scene), 8 KV / 32 query
    heads, 4-bit g64.  Timed twice, single-threaded and on `threads` OpenMP
    threads, each repeated until at least `min_seconds` of wall time."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    H, Hq, D = 8, 32, 128
    lens = (np.random.default_rng(3).integers(128, 8193, 64) + 1).astype(np.int32)
    rows = lens.astype(np.int64) * H          # [H, T] rows per sequence
    tok_off = np.concatenate([[0], np.cumsum(rows)[:-1]]).astype(np.int64)
    total = int(rows.sum())
    # quantize a 64K-row random pool, then tile it: values do not change
    # the oracle's running time
    rng = np.random.default_rng(5)
    pool = O.from_f32(rng.standard_normal((65536, D)).astype(np.float32), O.BF16)
    kq0, ks0, kb0, _ = O.quantize(pool, O.BF16, 64, 4)
    vq0, vs0, vb0, _ = O.quantize(pool[::-1].copy(), O.BF16, 64, 4)
    f = lambda a: O.to_f32(a, O.BF16)
    tile = lambda a: np.resize(a, (total,) + a.shape[1:])
    kq, vq = tile(kq0), tile(vq0)
    ks, kb, vs, vb = tile(f(ks0)), tile(f(kb0)), tile(f(vs0)), tile(f(vb0))
    q = f(O.from_f32(rng.standard_normal((len(lens), Hq, D)).astype(np.float32), O.BF16))
    layer_bytes = int(lens.sum()) * H * BYTES_PER_TOKEN_HEAD

    def run(n_threads):
        passes = 0
        t0 = time.perf_counter()
        while True:
            O.quantized_decode_batch(q, O.BF16, kq, ks, kb, vq, vs, vb, lens, tok_off, H,
                                     D ** -0.5, 64, 4, threads=n_threads,
                                     rounding=O.REF_DECODE)
            passes += 1
            dt = time.perf_counter() - t0
            if dt >= min_seconds:
                return passes * layer_bytes / dt / 1e9, passes, dt

    one, p1, t1 = run(1)
    many, pn, tn = run(threads)
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return {"value": round(many, 4), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "single_thread": {"value": round(one, 4), "unit": "GB/s", "cores": 1},
            "host_cpus": {"nproc": avail, "os_cpu_count": os.cpu_count()},
            "sample": f"one config-3 layer: 64 sequences ({int(lens.sum())} tokens) x 8 KV / 32 "
                      f"query heads, 4-bit g64; C oracle (restatement of the reference "
                      f"arithmetic, fp64 accumulation); {threads} OpenMP threads: {pn} passes "
                      f"in {tn:.1f} s; 1 thread: {p1} passes in {t1:.1f} s"}


F32_VALU_PEAK_TFLOPS = 157.3  # MI355X dense fp32 (vector and matrix)


def turboquant_measure(torch, vkv, steps, warmup):
    """TurboQuantKVCache.fromSimpleCache at a Llama-3-8B layer's shape
    (config 2: B 8, 8 KV heads x 128, 4096 bf16 tokens) with the reference's
    defaults (keyBits 3, valueBits 3, 4 sink and 64 residual tokens): encode
    K and V, decode both once into the unified buffer.  The key kernels
    dominate: each vector's QJL projection (encode) and sign product
    (decode) is a 128 x 128 f32 matrix-vector product, 2 * 128^2 flops."""
    B, H, T, D = 8, 8, 4096, 128
    bf = dict(dtype=torch.bfloat16, device="cuda")
    k = vkv.fill_normal(torch.empty((B, H, T, D), **bf), 61)
    v = vkv.fill_normal(torch.empty((B, H, T, D), **bf), 62)
    simple = vkv.KVCacheSimple()
    simple.update(k, v)
    keep = []

    def compress():
        keep.append(vkv.TurboQuantKVCache.from_simple_cache(simple, 3, 3))
        if len(keep) > 2:
            keep.pop(0)

    ms, enc_ms, enc_n = _time_calls(torch, vkv, compress, steps, warmup, vkv.TIME_TQ_ENCODE)
    vkv.kernel_timing(True)
    for _ in range(steps):
        compress()
    dec_ms, dec_n = vkv.kernel_timing_read(vkv.TIME_TQ_DECODE)
    vkv.kernel_timing(False)
    dec_ms /= max(dec_n, 1)
    rows = B * H * (T - 4 - 64)
    flops = rows * 2 * D * D
    enc_tf = flops / (enc_ms * 1e-3) / 1e12
    dec_tf = flops / (dec_ms * 1e-3) / 1e12
    sk, _ = keep[-1].state
    if not bool(torch.isfinite(sk.float()).all()):
        raise RuntimeError("the decoded TurboQuant keys hold non-finite values")
    return {
        "workload": "TurboQuantKVCache.fromSimpleCache, bf16 [8, 8, 4096, 128] K and V, keyBits 3, "
                    "valueBits 3, 4 sink + 64 residual tokens (encode + one decode, per layer)",
        "compress_ms_per_layer": round(ms, 4),
        "tokens_per_s": round(B * T / (ms * 1e-3), 1),
        "key_encode_kernel_us": round(enc_ms * 1e3, 2),
        "key_decode_kernel_us": round(dec_ms * 1e3, 2),
        "roofline": {"bound": "valu", "achieved": round(enc_tf, 2), "peak": F32_VALU_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(enc_tf / F32_VALU_PEAK_TFLOPS, 4),
                     "kernel": "tq_encode_rows<128, keys>", "flops_per_launch": flops},
        "decode_roofline": {"achieved": round(dec_tf, 2), "peak": F32_VALU_PEAK_TFLOPS,
                            "unit": "TFLOP/s", "frac": round(dec_tf / F32_VALU_PEAK_TFLOPS, 4),
                            "kernel": "tq_decode_rows<128, keys>"},
    }


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU: every GPU box in this build has one, "
              "so --gpus must be 1", file=sys.stderr)
        sys.exit(2)
    import torch

    import vkv

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    torch.cuda.set_device(0)
    if args.calibrate_copy:
        calibrate_copy(torch, vkv)
        return
    legs = {
        "config1": lambda: config1_measure(torch, vkv, args.steps, args.warmup),
        "config2": lambda: {f"bits{b}{sfx}": config2_measure(torch, vkv, args.steps, args.warmup,
                                                             b, ref)
                            for b in (4, 8) for ref, sfx in ((0, ""), (1, "_reference_softmax"))},
        "config4": lambda: config4_measure(torch, vkv, args.steps, args.warmup),
        "mla": lambda: mla_measure(torch, vkv, args.steps, args.warmup),
        "prefill": lambda: prefill_measure(torch, vkv, args.steps, args.warmup),
        "turboquant": lambda: turboquant_measure(torch, vkv, args.steps, args.warmup),
    }
    if args.only in legs:
        print(json.dumps({args.only: legs[args.only]()}), flush=True)
        return
    layers = args.layers
    pool, sc = build_scene(torch, vkv, layers)
    stream = torch.cuda.current_stream()
    scale = sc["D"] ** -0.5

    def step(ev=None):
        for l in range(layers):
            if ev is not None:
                ev[0][l].record(stream)
            pool.append(l, sc["ak"][l], sc["av"][l], sc["all_slots"])
            if ev is not None:
                ev[1][l].record(stream)
            o = sc["out"][l]
            vkv._chk(vkv.lib().vkv_paged_sdpa(
                vkv.C.byref(vkv.arr(sc["q"][l])), vkv.C.byref(sc["views"][l]), vkv.C.c_float(scale),
                vkv.C.byref(vkv.arr(o)), vkv.stream_ptr()))
            if ev is not None:
                ev[2][l].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # whole-step timing
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(args.steps):
        step()
    t1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / args.steps
    # per-kernel timing inside the same kind of steps
    # and the decode kernel alone (the attention call less its split-K
    # merge), from the library's event pair around that kernel
    app_ms = att_ms = 0.0
    for _ in range(args.steps):
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(layers)] for _ in range(3)]
        step(ev)
        torch.cuda.synchronize()
        for l in range(layers):
            app_ms += ev[0][l].elapsed_time(ev[1][l])
            att_ms += ev[1][l].elapsed_time(ev[2][l])
    vkv.kernel_timing(True)   # a pass of its own: the extra events add gaps
    for _ in range(args.steps):
        step()
    dec_ms, dec_n = vkv.kernel_timing_read(vkv.TIME_DECODE)
    appk_ms, appk_n = vkv.kernel_timing_read(vkv.TIME_APPEND)
    vkv.kernel_timing(False)
    torch.cuda.synchronize()
    if not bool(torch.isfinite(sc["out"].float()).all()):
        raise RuntimeError("the decode attention output holds non-finite values")
    # the attention calls alone with the reference softmax (score pass,
    # softmax pass, P.V pass, merge), for its cost against the fused call
    def att_only():
        for l in range(layers):
            vkv._chk(vkv.lib().vkv_paged_sdpa(
                vkv.C.byref(vkv.arr(sc["q"][l])), vkv.C.byref(sc["views"][l]), vkv.C.c_float(scale),
                vkv.C.byref(vkv.arr(sc["out"][l])), vkv.stream_ptr()))
    att_fused_ms, _, _ = _time_calls(torch, vkv, att_only, args.steps, args.warmup)
    vkv.set_option("reference_softmax", 1)
    try:
        att_ref_ms, _, _ = _time_calls(torch, vkv, att_only, args.steps, args.warmup)
    finally:
        vkv.set_option("reference_softmax", 0)
    att_fused_ms /= layers
    att_ref_ms /= layers
    n_att = args.steps * layers
    att_avg_ms = att_ms / n_att
    app_avg_ms = app_ms / n_att
    dec_avg_ms = dec_ms / max(dec_n, 1)
    appk_avg_ms = appk_ms / max(appk_n, 1)

    lens = sc["lens"] + 1
    logical = int(lens.sum()) * sc["H"] * BYTES_PER_TOKEN_HEAD
    unique = logical - (len(sc["sharers"]) - 1) * sc["share_tokens"] * sc["H"] * BYTES_PER_TOKEN_HEAD
    gbs_step = logical * layers / (ms_per_step * 1e-3) / 1e9
    att_gbs = logical / (att_avg_ms * 1e-3) / 1e9
    dec_gbs = logical / (dec_avg_ms * 1e-3) / 1e9
    append_tokens = sc["n_seqs"] + sc["prefill"]
    others = args.only == "all" and not args.no_mla
    mla = legs["mla"]() if others else None
    prefill = legs["prefill"]() if others else None
    configs = ({k: legs[k]() for k in ("config1", "config2", "config4", "turboquant")}
               if others else None)
    cpu = None
    if not args.no_cpu_baseline and args.only == "all":
        # all the host CPUs this process may use, at most 16 (a GPU box's
        # share of its host)
        try:
            avail = len(os.sched_getaffinity(0))
        except AttributeError:
            avail = os.cpu_count() or 1
        threads = args.cpu_threads or min(16, avail)
        cpu = cpu_baseline(threads)
    rec = {
        "metric": "KV-read GB/s (% HBM peak) in paged quant decode attn; KV append tokens/s",
        "value": round(gbs_step, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 KV stored affine u4 g64 (fp32 accumulate)",
        "data": "synthetic (GPU counter-based normal samples)",
        "config": {
            "workload": "paged continuous batching: 64 seqs U[128,8192] + 1 decode token, "
                        "pool 16384 x 32-token blocks per layer, 32/8 heads x 128, 4-bit g64, "
                        "32 seqs share a 2048-token prefix, +512-token chunked prefill append",
            "layers": layers, "n_seqs": sc["n_seqs"], "sum_len": int(lens.sum()),
            "kv_bytes_logical_per_layer": logical, "kv_bytes_unique_per_layer": unique,
        },
        "attention": {"ms_per_layer": round(att_avg_ms, 5), "gbs_logical": round(att_gbs, 1),
                      "gbs_unique": round(unique / (att_avg_ms * 1e-3) / 1e9, 1),
                      "pct_hbm_peak": round(100 * att_gbs / HBM_PEAK_GBS, 2),
                      "decode_kernel_ms": round(dec_avg_ms, 5),
                      "calls_back_to_back_ms_per_layer": round(att_fused_ms, 5),
                      "pct_hbm_peak_back_to_back": round(
                          100 * logical / (att_fused_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2)},
        "attention_reference_softmax": {
            "ms_per_layer": round(att_ref_ms, 5),
            "gbs_logical": round(logical / (att_ref_ms * 1e-3) / 1e9, 1),
            "pct_hbm_peak": round(100 * logical / (att_ref_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
            "note": "reference_softmax option: bf16 score rows, the reference's AccT = bf16 "
                    "softmax pass, P.V from the stored weights (calls back to back)"},
        # tokens/s over the append kernel's own time (its start/stop event
        # pair), and over the HIP events around the whole call
        "append": {"tokens_per_layer_step": append_tokens,
                   "kernel_ms_per_layer": round(appk_avg_ms, 5),
                   "tokens_per_s": round(append_tokens / (appk_avg_ms * 1e-3), 1),
                   "ms_per_layer_call": round(app_avg_ms, 5),
                   "tokens_per_s_call": round(append_tokens / (app_avg_ms * 1e-3), 1)},
        "roofline": {"bound": "hbm", "achieved": round(dec_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(dec_gbs / HBM_PEAK_GBS, 4),
                     "traffic": pmc_traffic(), "kernel": "qdecode_kernel",
                     "scope": "one decode launch, its split-K merge included"},
        "cpu_baseline": cpu,
        "mla": mla,
        "prefill": prefill,
        "configs": configs,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
