"""Benchmark of the speculative-decoding hot path on one MI355X.

Headline (`value`): emitted tokens/s of greedy speculative decoding at batch 1
with k = 4 and paged KV (block size 16), target with SmolLM2-1.7B shapes and
draft with SmolLM2-135M shapes, random-init bf16 weights, a 256-token seeded
prompt and 128 new tokens.  One step = one `generate` call.

`roofline`: the verify paged-attention kernel at B = 8, context 4096, 32/32
heads of 64, 5 query tokens, shuffled block table (config 2's largest
batch): algorithmic bytes per launch (K+V of 8 x 4101 positions + Q in + O
out + block tables) over the mean launch time measured with HIP events on
the stream it runs on.  B = 1 sits beside it in the line.

`cpu_baseline`: the oracle's CPU restatement of the reference loop
(gather + SDPA forward, host accept-reject) on the same weights, timed on a
bounded sample of the same request.

`kernels`: per-kernel times for the other workloads (accept-reject at
V = 49152, n-gram lookup at batch 16, cache append/rollback, attention over
the batch x context grid), each with its algorithmic bytes and GB/s.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only e2e|attention|kernels]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "speculative-decoder_amd"))

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the B=8, context-4096 verify attention (one tiled
# launch): rocprofv3 FETCH_SIZE + WRITE_SIZE of `bench.py --only attention`,
# each scaled by what the counter reads for a copy of known size.
ATTN_B8_TRAFFIC = 270_661_099
V = 49152
PROMPT = 256
NEW_TOKENS = 128
K = 4
BLOCK = 16


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ----------------------------------------------------------------- models ---
def build_models(dtype=torch.bfloat16, seed=0):
    from lm.model import SMOLLM2_135M, SMOLLM2_1_7B, Llama, random_state_dict

    dev = torch.device("cuda", 0)
    t_state = random_state_dict(SMOLLM2_1_7B, seed, dev, dtype)
    d_state = random_state_dict(SMOLLM2_135M, seed + 1, dev, dtype)
    return (Llama.from_state_dict(SMOLLM2_1_7B, t_state), Llama.from_state_dict(SMOLLM2_135M, d_state),
            t_state, d_state)


def mean_accept_len(stats):
    """Accepted draft tokens per (sequence, round)."""
    return stats.accepted / max(len(stats.emitted_per_round), 1)


def prompt_ids(seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, V, (PROMPT,), generator=g).tolist()


def make_caches(target, draft, new_tokens=NEW_TOKENS):
    """Target and draft caches sized for one request; reused across requests
    (sequences are freed at the end of each), as a server would."""
    from cache.kv import KVCache

    blocks = (PROMPT + new_tokens + 2 * K + 2 * BLOCK) // BLOCK + 4
    return (KVCache.for_model(target.config, blocks, BLOCK, target.dtype, "cuda"),
            KVCache.for_model(draft.config, blocks, BLOCK, draft.dtype, "cuda"))


def run_e2e(target, draft, prompt, caches, new_tokens=NEW_TOKENS):
    from spec.draft import ModelDraft
    from spec.loop import generate

    tc, dc = caches
    out, stats = generate(target, tc, ModelDraft(draft, dc), [prompt], new_tokens, k=K,
                          generator=torch.Generator().manual_seed(0))
    return out[0], stats


def bench_e2e(steps, warmup):
    target, draft, t_state, d_state = build_models()
    prompt = prompt_ids()
    caches = make_caches(target, draft)
    log("e2e warmup")
    for _ in range(warmup):
        run_e2e(target, draft, prompt, caches)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    outs = []
    for _ in range(steps):
        out, stats = run_e2e(target, draft, prompt, caches)
        outs.append(out)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    emitted = sum(len(o) for o in outs)
    result = {"tokens_per_s": emitted / dt, "ms_per_step": 1000 * dt / steps, "emitted_per_step": len(outs[0]),
              "rounds": stats.rounds, "mean_accept_len": mean_accept_len(stats),
              "acceptance": stats.accepted / max(stats.drafted, 1)}
    # identity check of this output against plain greedy decoding of the target
    from baselines.cached_autoregressive import generate as plain
    from cache.kv import KVCache

    blocks = (PROMPT + NEW_TOKENS + 2 * BLOCK) // BLOCK + 4
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    want = plain(target, KVCache.for_model(target.config, blocks, BLOCK, target.dtype, "cuda"), prompt, NEW_TOKENS)
    torch.cuda.synchronize()
    result["plain_greedy_tokens_per_s"] = NEW_TOKENS / (time.perf_counter() - t1)
    result["identical_to_plain_greedy"] = want == outs[0]
    result["first_divergence"] = next((i for i, (a, b) in enumerate(zip(want, outs[0])) if a != b), None)
    return result, (target, draft, t_state, d_state, prompt, outs[0])


def bench_variant_b(target, t_state, prompt, steps=1, n_layers=4, noise=0.002):
    """Config 4, second variant: the draft is the target's first `n_layers`
    layers (embeddings, final norm and head shared) plus N(0, noise^2) on
    every matrix of those layers."""
    from cache.kv import KVCache
    from lm.model import SMOLLM2_1_7B, Llama, perturbed_truncation
    from spec.draft import ModelDraft
    from spec.loop import generate

    state, shape = perturbed_truncation(t_state, SMOLLM2_1_7B, n_layers, noise, seed=7)
    draft = Llama.from_state_dict(shape, state)
    blocks = (PROMPT + NEW_TOKENS + 2 * K + 2 * BLOCK) // BLOCK + 4
    tc = KVCache.for_model(target.config, blocks, BLOCK, target.dtype, "cuda")
    dc = KVCache.for_model(draft.config, blocks, BLOCK, draft.dtype, "cuda")
    generate(target, tc, ModelDraft(draft, dc), [prompt], NEW_TOKENS, k=K, generator=torch.Generator().manual_seed(0))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out, stats = generate(target, tc, ModelDraft(draft, dc), [prompt], NEW_TOKENS, k=K,
                              generator=torch.Generator().manual_seed(0))
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    return {"draft": f"target layers 0..{n_layers - 1} + N(0, {noise}^2)", "tokens_per_s": len(out[0]) / dt,
            "acceptance": stats.accepted / max(stats.drafted, 1),
            "mean_accept_len": mean_accept_len(stats), "rounds": stats.rounds}


def bench_batched(target, draft, combos=((8, 4, "model"), (8, 4, "ngram"), (32, 8, "model"), (32, 8, "ngram")),
                  prompt_len=1024, new_tokens=32, temperature=0.8):
    """Config 5, bounded: batched sampled speculative decoding on seeded
    1024-token prompts with ~30% planted repetition, `new_tokens` per row.
    Reports emitted tokens/s, mean accept length, and per round the accept
    kernel time (HIP events around the call the loop makes) and the verify
    attention kernel time at that batch and context (graph-replayed)."""
    import spec.loop as loop_mod
    from cache.kv import KVCache
    from specdec.workloads import planted_rows
    from spec.draft import ModelDraft
    from spec.loop import generate
    from spec.ngram import NGramDraft

    results = {}
    for batch, k, kind in combos:
        prompts = planted_rows(batch, prompt_len, V, seed=batch * 100 + k)
        blocks = batch * ((prompt_len + new_tokens + 2 * k + 2 * BLOCK) // BLOCK + 2) + 8
        tc = KVCache.for_model(target.config, blocks, BLOCK, target.dtype, "cuda", )
        dc = KVCache.for_model(draft.config, blocks, BLOCK, draft.dtype, "cuda") if kind == "model" else None
        accept_us = []
        real_accept = loop_mod.accept_reject

        def timed_accept(*a, **kw):
            st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            st.record()
            v = real_accept(*a, **kw)
            en.record()
            en.synchronize()
            accept_us.append(st.elapsed_time(en) * 1000)
            return v

        def run():
            drafter = ModelDraft(draft, dc) if kind == "model" else NGramDraft(V)
            return generate(target, tc, drafter, prompts, new_tokens, k=k, temperature=temperature,
                            generator=torch.Generator().manual_seed(5))

        run()  # warm-up: captures the graphs of this shape
        loop_mod.accept_reject = timed_accept
        try:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            outs, stats = run()
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
        finally:
            loop_mod.accept_reject = real_accept
        attn = time_attention(batch, prompt_len + new_tokens // 2, iters=40, t_new=k + 1)
        results[f"b{batch}_k{k}_{kind}"] = {
            "tokens_per_s": sum(len(o) for o in outs) / dt, "mean_accept_len": mean_accept_len(stats),
            "acceptance": stats.accepted / max(stats.drafted, 1),
            "rounds": stats.rounds, "accept_call_us_per_round": sum(accept_us) / max(len(accept_us), 1),
            "verify_attention_us_per_layer": attn["us"], "verify_attention_gbs": attn["gbs"],
            "sample": f"{batch} rows, {prompt_len}-token prompts (~30% planted repetition), {new_tokens} new tokens, "
                      f"T={temperature}, k={k}"}
        log(f"batched {batch} {k} {kind}: {results[f'b{batch}_k{k}_{kind}']}")
        del tc, dc
        torch.cuda.empty_cache()
    return results


# ------------------------------------------------------------ attention -----
def attention_bytes(batch, lengths, t_new=5, h=32, hkv=32, d=64, bs=BLOCK):
    kv = sum((L + t_new) * hkv * d * 2 * 2 for L in lengths)
    qo = batch * t_new * h * d * 2 * 2
    tables = sum(-(-(L + t_new) // bs) * 4 for L in lengths)
    return kv + qo + tables


def setup_attention(batch, length, seed=0, h=32, hkv=32, d=64, t_new=5, num_blocks=4096, layers=1):
    """Config 2: pool of 4096 blocks handed out in a seeded random order,
    `length` cached positions per row, then an append of t_new tokens.
    `layers` pools share the block table, as the layers of a model do."""
    from cache.kv import KVCache

    need = batch * (-(-(length + t_new) // BLOCK))
    num_blocks = max(num_blocks, need + 8)
    cache = KVCache(layers, hkv, d, num_blocks, BLOCK, torch.bfloat16, "cuda", max_seqs=batch + 2)
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(seed))
    cache.add(-1)
    cache.append([-1], [num_blocks * BLOCK])
    cache.table_tensor[cache.tables[-1].row, :num_blocks] = perm.to(torch.int32).cuda()
    cache.free(-1)
    cache.flush()
    ids = list(range(batch))
    for s in ids:
        cache.add(s)
    g = torch.Generator(device="cuda").manual_seed(seed)
    step = cache.append(ids, [length] * batch)
    cache.k.normal_(generator=g)
    cache.v.normal_(generator=g)
    step = cache.append(ids, [t_new] * batch)
    q = torch.randn(batch, t_new, h * d, generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty_like(q)
    return cache, step, q, out


def graph_time_us(launch, per_graph=20, replays=10):
    """Mean GPU time of `launch` (one kernel) from HIP events around replays of
    a graph holding `per_graph` back-to-back launches, so host launch cost
    is not in the measurement."""
    for _ in range(3):
        launch()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_graph):
            launch()
    graph.replay()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    stream.synchronize()
    start.record(stream)
    for _ in range(replays):
        graph.replay()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) * 1000 / (per_graph * replays)


MALL_BYTES = 256 << 20  # MI355X last-level (Infinity) cache


def attention_layers(batch, length, t_new=5, hkv=32, d=64):
    """Layer pools to cycle through so that the K/V read by consecutive
    launches exceed the last-level cache at least threefold: every launch
    then reads HBM, as the layers of a 24-layer model do."""
    touched = batch * (length + t_new) * hkv * d * 2 * 2
    return min(24, max(2, -(-3 * MALL_BYTES // touched)))


def time_attention(batch, length, iters=200, t_new=5, rotate=True):
    """Verify attention over the config-2 setup.  With `rotate`, launches
    cycle over attention_layers() layer pools (K/V from HBM); without, they
    re-read one pool, which at batch 1 (34 MB) stays in the last-level cache."""
    from specdec import ops

    layers = attention_layers(batch, length, t_new) if rotate else 1
    cache, step, q, out = setup_attention(batch, length, t_new=t_new, layers=layers)
    h, hkv, d = 32, 32, 64
    ws = ops.AttentionWorkspace(q.device)
    turn = [0]

    def launch():
        i = turn[0] % layers
        turn[0] += 1
        ops.paged_attention(q, q.stride(1), cache.k[i], cache.v[i], cache.table_tensor, step.meta, batch, t_new, h,
                            hkv, d, BLOCK, 0.125, step.max_total, out, out.stride(1), ws)

    launch()
    per_graph = layers * -(-20 // layers)
    us = graph_time_us(launch, per_graph=per_graph, replays=max(iters // per_graph, 2))
    nbytes = attention_bytes(batch, [length] * batch, t_new=t_new)
    del cache
    torch.cuda.empty_cache()
    return {"batch": batch, "context": length, "us": us, "bytes": nbytes, "gbs": nbytes / us / 1e3,
            "frac_of_peak": nbytes / us / 1e3 / HBM_PEAK_GBS, "layer_pools": layers,
            "kv_source": "HBM (layer pools cycled)" if rotate else "one pool re-read"}


# ------------------------------------------------------- other kernels ------
def time_fn(fn, iters=100, graph=False):
    if graph:
        return graph_time_us(fn, per_graph=10, replays=max(iters // 10, 1))
    for _ in range(5):
        fn()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    stream.synchronize()
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) * 1000 / iters


def bench_kernels(attention_grid=True):
    from specdec.workloads import planted_rows
    from specdec import ops

    res = {}
    # config 1: accept-reject, B=1, k=4, V=49152, fp32, T=1
    for b, k in [(1, 4), (8, 4), (32, 8)]:
        g = torch.Generator(device="cuda").manual_seed(1)
        tl = torch.randn(b, k + 1, V, generator=g, device="cuda") * 2
        dl = tl[:, :k] + torch.randn(b, k, V, generator=g, device="cuda") * 0.5
        p = ops.probabilities(tl, 1.0)
        q = ops.probabilities(dl, 1.0)
        draft = torch.randint(0, V, (b, k), device="cuda")
        q.view(-1, V)[torch.arange(b * k, device="cuda"), draft.view(-1)] += 1e-3
        ua = torch.rand(b, k, generator=g, device="cuda")
        ur = torch.rand(b, generator=g, device="cuda")
        both = torch.cat([tl.view(-1, V), dl.view(-1, V)])
        us_soft = time_fn(lambda: ops.probabilities(both, 1.0), graph=True)
        us_acc = time_fn(lambda: ops.accept_reject(p, q, draft, ua, ur), graph=True)
        logit_bytes = (2 * k + 1) * V * 4 * b
        # the accept kernel reads the rejected position's p and q rows (and
        # gathers 2k probabilities): 2 V fp32 per batch entry
        accept_bytes = 2 * V * 4 * b
        res[f"accept_b{b}_k{k}"] = {"softmax_us": us_soft, "accept_us": us_acc, "logit_bytes": logit_bytes,
                                    "softmax_gbs": 2 * logit_bytes / us_soft / 1e3,
                                    "softmax_frac_of_peak": 2 * logit_bytes / us_soft / 1e3 / HBM_PEAK_GBS,
                                    "accept_bytes": accept_bytes, "accept_gbs": accept_bytes / us_acc / 1e3,
                                    "accept_frac_of_peak": accept_bytes / us_acc / 1e3 / HBM_PEAK_GBS}
    # config 3: n-gram, B=16
    for length in (2048, 4096, 8192):
        rows = planted_rows(16, length, V, seed=length)
        hist = torch.tensor(rows, dtype=torch.int32, device="cuda")
        lens = torch.full((16,), length, dtype=torch.int32, device="cuda")
        us = time_fn(lambda: ops.ngram_lookup(hist, lens, 4, 3), graph=True)
        nbytes = 16 * length * 4
        res[f"ngram_b16_L{length}"] = {"us": us, "bytes": nbytes, "gbs": nbytes / us / 1e3,
                                       "frac_of_peak": nbytes / us / 1e3 / HBM_PEAK_GBS}
    # config 2': cache append (rope + scatter of 5 tokens) and rollback plan
    cache, step, q, out = setup_attention(1, 4096)
    qkv = torch.randn(1, 5, 96 * 64, device="cuda").to(torch.bfloat16)
    from lm.model import SMOLLM2_1_7B, rope_tables

    cos, sin = (t.cuda() for t in rope_tables(SMOLLM2_1_7B, 8192))
    us_app = time_fn(lambda: ops.rope_append(qkv, 32, 32, 64, cos, sin, step.meta, 1, 5, cache.table_tensor, BLOCK,
                                             cache.k[0], cache.v[0]), graph=True)
    app_bytes = 5 * 96 * 64 * 2 + 5 * 64 * 64 * 2
    res["append_b1_t5"] = {"us": us_app, "bytes": app_bytes, "gbs": app_bytes / us_app / 1e3,
                           "frac_of_peak": app_bytes / us_app / 1e3 / HBM_PEAK_GBS}
    # config 2': one round's rollback of 8 rows (a rejected tail each) and the
    # regrowth for the next verify: the block plan the cache launches
    ids = list(range(8))
    cache8, _, _, _ = setup_attention(8, 1005)  # 1010 cached: the rollback frees a block, the regrowth takes one
    lens = [cache8.length(s) for s in ids]

    def rollback_and_grow():
        for s, n in zip(ids, lens):
            cache8.truncate(s, n - 5 + 1)
        cache8.append(ids, [4] * 8)

    res["rollback_grow_b8"] = {"us_host_inclusive": time_fn(rollback_and_grow, iters=50)}
    del cache8
    if not attention_grid:
        return res
    # attention over the config-2 grid
    for b in (1, 4, 8):
        for L in (512, 1024, 2048, 4096):
            res[f"attention_b{b}_L{L}"] = time_attention(b, L, iters=50)
    return res


# ------------------------------------------------------------ CPU side ------
def cpu_baseline(t_state, d_state, prompt, new_tokens=64):
    """Oracle loop on the host cores: same weights (bf16), same prompt, a
    bounded number of new tokens."""
    import oracle.forward as of
    import oracle.kv as okv
    from lm.model import SMOLLM2_135M, SMOLLM2_1_7B
    from oracle.draft import ModelDraft
    from oracle.loop import generate

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)

    def cfg(s):
        return of.Config(s.vocab_size, s.hidden_size, s.num_hidden_layers, s.num_attention_heads,
                         s.num_key_value_heads, s.intermediate_size, s.head_dim, s.rms_norm_eps, s.rope_theta, True)

    tm = of.Model(cfg(SMOLLM2_1_7B), {k: v.cpu() for k, v in t_state.items()})
    dm = of.Model(cfg(SMOLLM2_135M), {k: v.cpu() for k, v in d_state.items()})
    blocks = (PROMPT + new_tokens + 2 * K + 2 * BLOCK) // BLOCK + 4
    t0 = time.perf_counter()
    out, stats = generate(tm, okv.KVCache.for_model(tm.config, blocks, BLOCK, torch.bfloat16),
                          ModelDraft(dm, okv.KVCache.for_model(dm.config, blocks, BLOCK, torch.bfloat16)),
                          [prompt], new_tokens, K, generator=torch.Generator().manual_seed(0))
    dt = time.perf_counter() - t0
    return {"value": len(out[0]) / dt, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"oracle loop (gather+SDPA forward, CPU accept-reject), 256-token prompt, "
                      f"{new_tokens} new tokens, bf16, torch threads={threads}",
            "seconds": dt, "tokens": out[0]}


def cpu_attention_baseline(length=4096, batch=1, seconds=3.0):
    """Oracle attention step (gather copy + masked SDPA) at context 4096 on the CPU."""
    import oracle.forward as of

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    pool = torch.randn(4096 * BLOCK, 32, 64, generator=g).to(torch.bfloat16)
    nblk = -(-(length + 5) // BLOCK)
    perm = torch.randperm(4096, generator=g)[: batch * nblk].view(batch, nblk)
    read = (perm[:, :, None] * BLOCK + torch.arange(BLOCK)).flatten(1)[:, : length + 5]
    q = torch.randn(batch, 32, 5, 64, generator=g).to(torch.bfloat16)
    past, total = torch.full((batch,), length), torch.full((batch,), length + 5)
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        k_all = pool[read].transpose(1, 2)
        v_all = pool[read].transpose(1, 2)
        of.attention(q, k_all, v_all, past, total, 0.125)
        n += 1
    us = (time.perf_counter() - t0) / n * 1e6
    return {"us": us, "gbs": attention_bytes(batch, [length] * batch) / us / 1e3, "cores": threads}


def cpu_kernel_baselines(seconds=1.0):
    """The oracle (the reference's algorithms in torch on the host cores) on
    the kernels' own workloads, each repeated for about `seconds`:
    temperature softmax and accept-reject (config 1 and batch 8), n-gram
    lookup (config 3), and the cache's append + rollback bookkeeping
    (config 2': slot maps and block tables for 8 rows, one layer's write of
    5 tokens)."""
    import oracle.accept as oa
    import oracle.kv as okv
    import oracle.ngram as on
    import oracle.sampling as osamp
    from specdec.workloads import planted_rows

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)

    def timed(fn):
        fn()
        n, t0 = 0, time.perf_counter()
        while n == 0 or time.perf_counter() - t0 < seconds:
            fn()
            n += 1
        return (time.perf_counter() - t0) / n * 1e6

    res = {"cores": threads}
    for b, k in ((1, 4), (8, 4)):
        g = torch.Generator().manual_seed(1)
        tl = torch.randn(b, k + 1, V, generator=g) * 2
        dl = tl[:, :k] + torch.randn(b, k, V, generator=g) * 0.5
        p, q = osamp.probabilities(tl, 1.0), osamp.probabilities(dl, 1.0)
        draft = torch.randint(0, V, (b, k), generator=g)
        ua, ur = torch.rand(b, k, generator=g), torch.rand(b, generator=g)
        both = torch.cat([tl.reshape(-1, V), dl.reshape(-1, V)])
        res[f"softmax_b{b}_k{k}_us"] = timed(lambda: osamp.probabilities(both, 1.0))
        res[f"accept_b{b}_k{k}_us"] = timed(lambda: oa.accept_reject(p, q, draft, u_accept=ua, u_residual=ur))
    for length in (2048, 4096, 8192):
        rows = planted_rows(16, length, V, seed=length)
        res[f"ngram_b16_L{length}_us"] = timed(lambda: [on.lookup_match(r, 4, 3) for r in rows])
    cache = okv.KVCache(1, 32, 64, 8 * 70, BLOCK, torch.bfloat16)
    ids = list(range(8))
    for s in ids:
        cache.add(s)
    cache.append(ids, [1010] * 8)

    def rollback_and_grow():
        for s in ids:
            cache.truncate(s, 1010 - 5 + 1)
        cache.append(ids, [4] * 8)

    res["rollback_grow_b8_us"] = timed(rollback_and_grow)
    one = okv.KVCache(1, 32, 64, 300, BLOCK, torch.bfloat16)
    one.add(0)
    one.append([0], [4096])
    kv_new = torch.randn(1, 32, 5, 64).to(torch.bfloat16)

    def append_write():
        one.truncate(0, 4096)
        slots = one.append([0], [5])
        one.write(0, slots, kv_new, kv_new)

    res["append_b1_t5_us"] = timed(append_write)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--only", choices=["all", "e2e", "batched", "attention", "kernels", "small", "copy"], default="all",
                    help="small: the kernels of configs 1-3 without the attention grid (for counter runs)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-batched", action="store_true")
    ap.add_argument("--batch", type=int, default=8, help="batch of the --only attention run")
    ap.add_argument("--one-pool", action="store_true", help="--only attention: re-read one layer pool")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only; --gpus {args.gpus} is not supported (the path is built and "
              "measured on a single GPU; sharding across GPUs is not implemented)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    sys.path.insert(0, str(ROOT))

    if args.only == "attention":
        r = time_attention(args.batch, 4096, iters=max(args.steps, 1) * 100, rotate=not args.one_pool)
        print(json.dumps({f"attention_b{args.batch}_L4096": r}))
        return
    if args.only in ("kernels", "small"):
        print(json.dumps(bench_kernels(attention_grid=args.only == "kernels")))
        return
    if args.only == "copy":
        # reference copy of a known size for scaling the FETCH_SIZE / WRITE_SIZE counters
        x = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        y = torch.empty_like(x)
        for _ in range(max(args.steps, 1)):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_each_way": x.numel() * 4, "launches": max(args.steps, 1)}))
        return
    if args.only == "e2e":
        e2e, _ = bench_e2e(args.steps, args.warmup)
        print(json.dumps({"e2e": e2e}))
        return
    if args.only == "batched":
        target, draft, _, _ = build_models()
        print(json.dumps({"batched_sampled": bench_batched(target, draft)}))
        return

    e2e, (target, draft, t_state, d_state, prompt, gpu_tokens) = bench_e2e(args.steps, args.warmup)
    log(f"e2e {e2e}")
    attn = time_attention(8, 4096, iters=120)
    log(f"attention b8 {attn}")
    attn1 = time_attention(1, 4096, iters=300)
    log(f"attention b1 {attn1}")
    attn1_pool = time_attention(1, 4096, iters=300, rotate=False)
    log(f"attention b1 one pool {attn1_pool}")
    kernels = {} if args.only == "e2e" else bench_kernels()
    variant_b = bench_variant_b(target, t_state, prompt)
    log(f"variant B {variant_b}")
    batched = {} if args.no_batched else bench_batched(target, draft)
    cpu = None
    if not args.no_cpu:
        del target, draft
        torch.cuda.empty_cache()
        log("cpu baseline")
        cpu = cpu_baseline(t_state, d_state, prompt)
        cpu_tokens = cpu.pop("tokens")
        # bf16 GEMMs round differently on the host and the GPU, so the two bf16
        # token streams may part; the fp32 identity against the oracle is a test
        cpu["bf16_first_divergence_from_gpu"] = next(
            (i for i, (x, y) in enumerate(zip(cpu_tokens, gpu_tokens)) if x != y), None)
        cpu["attention_b1_L4096"] = cpu_attention_baseline()
        cpu["attention_b8_L4096"] = cpu_attention_baseline(batch=8)
        cpu["kernels"] = cpu_kernel_baselines()
    line = {
        "metric": "spec-decode accepted tokens/s, 1.7B/135M k=4 b=1; verify-attn HBM GB/s",
        "value": e2e["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": e2e["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights N(0, 0.02), seeded uniform prompt ids)",
        "config": {"workload": "greedy speculative decode, target SmolLM2-1.7B shapes / draft SmolLM2-135M shapes, "
                               "batch 1, k=4, paged KV block 16, prompt 256, 128 new tokens",
                   "batch": 1, "k": K, "prompt": PROMPT, "new_tokens": NEW_TOKENS, "block_size": BLOCK},
        "roofline": {"bound": "hbm", "achieved": attn["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": attn["gbs"] / HBM_PEAK_GBS, "traffic": ATTN_B8_TRAFFIC,
                     "kernel": "verify paged attention (attention_bf16_kernel<1, 16, true>: one 16-wave workgroup "
                               "per (row, kv head) tile taking its 512-token splits in rounds, no combine launch), "
                               "B=8, context 4096 (+5 appended), 32/32 heads x 64, bf16, block 16, K/V from HBM",
                     "us_per_launch": attn["us"], "bytes_per_launch": attn["bytes"]},
        "cpu_baseline": cpu,
        "e2e": e2e,
        "e2e_variant_b": variant_b,
        "attention_b1_ctx4096": attn1,
        "attention_b1_ctx4096_one_pool": attn1_pool,
        "batched_sampled": batched,
        "kernels": kernels,
    }
    if cpu:
        line["cpu_baseline"]["speedup"] = e2e["tokens_per_s"] / cpu["value"]
        line["cpu_baseline"]["kernel_speedups"] = kernel_speedups(kernels, cpu, attn, attn1)
    print(json.dumps(line))


def kernel_speedups(kernels, cpu, attn8, attn1):
    """Host-oracle time over GPU time for each kernel timed on both sides."""
    ck = cpu.get("kernels", {})
    pairs = {"attention_b1_L4096": (cpu["attention_b1_L4096"]["us"], attn1["us"]),
             "attention_b8_L4096": (cpu["attention_b8_L4096"]["us"], attn8["us"])}
    for b, k in ((1, 4), (8, 4)):
        g = kernels.get(f"accept_b{b}_k{k}")
        if g:
            pairs[f"softmax_b{b}_k{k}"] = (ck[f"softmax_b{b}_k{k}_us"], g["softmax_us"])
            pairs[f"accept_b{b}_k{k}"] = (ck[f"accept_b{b}_k{k}_us"], g["accept_us"])
    for length in (2048, 4096, 8192):
        g = kernels.get(f"ngram_b16_L{length}")
        if g:
            pairs[f"ngram_b16_L{length}"] = (ck[f"ngram_b16_L{length}_us"], g["us"])
    if "append_b1_t5" in kernels:
        pairs["append_b1_t5"] = (ck["append_b1_t5_us"], kernels["append_b1_t5"]["us"])
    if "rollback_grow_b8" in kernels:
        pairs["rollback_grow_b8"] = (ck["rollback_grow_b8_us"], kernels["rollback_grow_b8"]["us_host_inclusive"])
    return {name: c / g for name, (c, g) in pairs.items()}


if __name__ == "__main__":
    main()
