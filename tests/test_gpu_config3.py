"""The paged continuous-batching workload at its full size, the scene the
benchmark times: a 16384-block pool of 32-token 4-bit g64 blocks, 64
sequences with lengths U[128, 8192] whose block tables are random
permutations of pool ids, 32 of them sharing one refcounted 2048-token
prefix; one step appends a decode token per sequence plus a 512-token
chunked-prefill chunk (one append call), then runs decode attention with 32
query heads over all 64 sequences.

Checked: the codes/scales/biases the append wrote for the shortest and the
longest sequence and two prefix sharers are bit-exact with the oracle
quantizer of the same bf16 inputs (regenerated from the counter-based
generator), the decode attention of those four sequences matches the
oracle with the reference's arithmetic (KVCache.swift:1909-1997), and every
output of the step is finite."""
import numpy as np
import pytest
import torch

import bench
import oracle as O
import vkv
from gpu_util import assert_qclose, host, qref, values

pytestmark = pytest.mark.gpu


def test_config3_full_scene_step_matches_oracle():
    print("config 3: building the full scene (1 layer)", flush=True)
    pool, sc = bench.build_scene(torch, vkv, 1)
    H, D, Hq, bs = sc["H"], sc["D"], sc["Hq"], sc["bs"]
    lens, sharers, share = sc["lens"], sc["sharers"], sc["share_tokens"]
    assert sc["n_seqs"] == 64 and sc["nblocks"] == 16384 and len(sharers) == 32
    # one step: the decode token of every sequence plus the prefill chunk
    pool.append(0, sc["ak"][0], sc["av"][0], sc["all_slots"])
    out = vkv.paged_attention(sc["q"][0], sc["views"][0], D ** -0.5)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all())
    # the fill inputs, regenerated: rows in sequence order, sharers after the
    # first skipping the shared prefix
    starts = [share if (s in sharers and s != sharers[0]) else 0 for s in range(64)]
    nfill = sum(int(lens[s]) - starts[s] for s in range(64))
    row0 = np.cumsum([0] + [int(lens[s]) - starts[s] for s in range(64)])
    stage = torch.empty((nfill, H, D), dtype=torch.bfloat16, device="cuda")
    fill = {}
    for which, seed in (("k", 1000), ("v", 1001)):
        vkv.fill_normal(stage, seed=seed)
        torch.cuda.synchronize()
        fill[which] = stage
        stage = torch.empty_like(stage)
    order = np.argsort(lens)
    picks = [int(order[0]), int(order[-1])]
    picks += [s for s in (sharers[1], sharers[-1], sharers[2], sharers[-2]) if s not in picks][:2]
    print(f"config 3: checking sequences {picks} (lengths {[int(lens[s]) for s in picks]})",
          flush=True)
    dtype = O.BF16
    f = lambda a: O.to_f32(a, dtype)
    q = host(sc["q"][0])
    got_all = values(out, dtype)
    for s in picks:
        L = int(lens[s]) + 1
        toks = {}
        for which, dec in (("k", sc["dk"]), ("v", sc["dv"])):
            src = fill[which]
            own = host(src[row0[s]:row0[s + 1]])
            if starts[s]:
                first = sharers[0]
                own = np.concatenate([host(src[row0[first]:row0[first] + share]), own])
            toks[which] = np.concatenate([own, host(dec[0, s:s + 1])])  # [L, H, D]
            assert toks[which].shape == (L, H, D)
        # the codes the append wrote, through a one-sequence view
        tab = sc["table"][s:s + 1]
        view = pool.view(0, tab, torch.tensor([L], dtype=torch.int32, device="cuda"), L)
        (kq, ks, kb), (vq, vs, vb) = vkv.paged_gather_quantized(view)
        ref_codes = []
        for which, got in (("k", (kq, ks, kb)), ("v", (vq, vs, vb))):
            x = np.ascontiguousarray(toks[which].transpose(1, 0, 2))  # [H, L, D]
            rq, rs, rb, _ = O.quantize(x, dtype, 64, 4)
            assert np.array_equal(host(got[0][0]), rq), (s, which)
            assert np.array_equal(host(got[1][0]).view(rs.dtype), rs), (s, which)
            assert np.array_equal(host(got[2][0]).view(rb.dtype), rb), (s, which)
            ref_codes.append((rq, rs, rb))
        (rkq, rks, rkb), (rvq, rvs, rvb) = ref_codes
        ref, wb = (x[0, :, 0] for x in qref(
            f(q[s])[None, :, None], dtype, rkq[None], f(rks)[None], f(rkb)[None], rvq[None],
            f(rvs)[None], f(rvb)[None], D ** -0.5, 64, 4))
        assert_qclose(got_all[s], ref, wb, dtype, f"sequence {s} (length {L})")
