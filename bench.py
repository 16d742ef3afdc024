"""Benchmark: paged 4-bit KV decode attention + KV append (config 3).

Workload ("Paged continuous batching"): a pool of
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
"attention" times the paged decode call (decode kernel + split-K merge),
"roofline" the decode kernel alone (the library's event pair around it, on
its launch stream), "traffic" is the PMC-measured HBM bytes per decode launch,
"cpu_baseline" times the C oracle, "prefill" times a 512-token chunked-prefill
attention step over a 4-bit cache, and "mla" is the MLA latent decode workload
(32 x 16384 tokens, 128 heads) with the MFMA roofline of its attention kernel.
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


def cpu_baseline(threads, min_seconds=10.0):
    """The CPU oracle (C restatement of the reference arithmetic, fp64,
    OpenMP) on one layer of the same workload: the 64 config-3 sequences
    (same lengths as the GPU scene), 8 KV / 32 query heads, 4-bit g64.
    Passes are repeated until at least `min_seconds` of CPU time."""
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
    passes = 0
    t0 = time.perf_counter()
    while True:
        O.quantized_decode_batch(q, O.BF16, kq, ks, kb, vq, vs, vb, lens, tok_off, H, D ** -0.5,
                                 64, 4, threads=threads)
        passes += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds:
            break
    byts = passes * int(lens.sum()) * H * BYTES_PER_TOKEN_HEAD
    return {"value": round(byts / dt / 1e9, 4), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"one config-3 layer: 64 sequences ({int(lens.sum())} tokens) x 8 KV / 32 "
                      f"query heads, 4-bit g64; {passes} passes in {dt:.1f} s; C oracle (fp64 "
                      f"restatement of the reference arithmetic, OpenMP, {threads} threads)"}


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
    vkv.kernel_timing(False)
    torch.cuda.synchronize()
    if not bool(torch.isfinite(sc["out"].float()).all()):
        raise RuntimeError("the decode attention output holds non-finite values")
    n_att = args.steps * layers
    att_avg_ms = att_ms / n_att
    app_avg_ms = app_ms / n_att
    dec_avg_ms = dec_ms / max(dec_n, 1)

    lens = sc["lens"] + 1
    logical = int(lens.sum()) * sc["H"] * BYTES_PER_TOKEN_HEAD
    unique = logical - (len(sc["sharers"]) - 1) * sc["share_tokens"] * sc["H"] * BYTES_PER_TOKEN_HEAD
    gbs_step = logical * layers / (ms_per_step * 1e-3) / 1e9
    att_gbs = logical / (att_avg_ms * 1e-3) / 1e9
    dec_gbs = logical / (dec_avg_ms * 1e-3) / 1e9
    append_tokens = sc["n_seqs"] + sc["prefill"]
    mla = None if args.no_mla else mla_measure(torch, vkv, args.steps, args.warmup)
    prefill = None if args.no_mla else prefill_measure(torch, vkv, args.steps, args.warmup)
    cpu = None
    if not args.no_cpu_baseline:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
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
                      "decode_kernel_ms": round(dec_avg_ms, 5)},
        "append": {"tokens_per_layer_step": append_tokens,
                   "ms_per_layer": round(app_avg_ms, 5),
                   "tokens_per_s": round(append_tokens / (app_avg_ms * 1e-3), 1)},
        "roofline": {"bound": "hbm", "achieved": round(dec_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(dec_gbs / HBM_PEAK_GBS, 4),
                     "traffic": pmc_traffic(), "kernel": "qdecode_kernel"},
        "cpu_baseline": cpu,
        "mla": mla,
        "prefill": prefill,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
