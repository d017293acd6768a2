"""Write golden input/output vectors by running the reference implementation
(beriltatli/speculative-decoder, read from /root/reference) in this
container, for the functions whose exact outputs no reference test fixes:

  accept_gen.json   accept_reject drawing its own uniforms from a seeded
                    generator (RNG order and dtype), fp32 and fp64
  ngram.json        lookup on config-3-like rows (planted copies, fallback)
  paged_ops.json    block ids, free-list order and stats under seeded
                    add/append/truncate/free sequences
  loop_tiny.json    spec.loop.generate on the reference's tiny fp64 model
                    (greedy and T=1), outputs and SpecStats

The reference is only imported here; nothing under tests/ reads
/root/reference at run time.  Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import random
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))
from workloads import accept_inputs, planted_rows  # noqa: E402

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent


def ref_import():
    sys.path.insert(0, str(REF))
    sys.path.insert(0, str(REF / "tests"))
    import spec.accept as accept  # noqa: E402
    import spec.ngram as ngram  # noqa: E402
    import cache.kv as kv  # noqa: E402

    return accept, ngram, kv


def make_accept(accept) -> dict:
    cases = []
    for case, (dtype, b, k, v, temp_noise) in enumerate(
            [(torch.float32, 6, 4, 64, 0.5), (torch.float64, 5, 3, 17, 1.0), (torch.float32, 8, 8, 256, 0.2),
             (torch.float32, 4, 4, 49152, 0.5)]):
        p, q, draft = accept_inputs(dtype, b, k, v, temp_noise, 100 + case)
        seed = 1000 + case
        verdict = accept.accept_reject(p, q, draft, generator=torch.Generator().manual_seed(seed))
        gu = torch.Generator().manual_seed(seed)
        ua = torch.rand(b, k, generator=gu, dtype=dtype)
        ur = torch.rand(b, generator=gu, dtype=dtype)
        cases.append({
            "dtype": str(dtype).replace("torch.", ""), "b": b, "k": k, "v": v, "seed": seed,
            # the probabilities themselves for small V; larger cases are
            # regenerated from input_seed by inputs() and checked by p_sha
            "p": p.tolist() if v <= 64 else None, "q": q.tolist() if v <= 64 else None,
            "input_seed": 100 + case, "noise": temp_noise,
            "draft": draft.tolist(), "u_accept": ua.tolist(), "u_residual": ur.tolist(),
            "n_accepted": verdict.n_accepted.tolist(), "next_token": verdict.next_token.tolist(),
            "p_sha": hashlib.sha256(p.numpy().tobytes()).hexdigest(),
        })
    return {"cases": cases}


def make_ngram(ngram) -> dict:
    cases = []
    for seed, (n_rows, length, vocab) in enumerate([(6, 64, 8), (6, 300, 50), (4, 2048, 49152), (3, 1, 10),
                                                   (3, 2, 5), (2, 5000, 49152)]):
        rows = planted_rows(n_rows, length, vocab, seed)
        for k in (1, 4, 6):
            for max_n in (1, 2, 3):
                cases.append({"rows": rows if length <= 300 else None, "gen": [n_rows, length, vocab, seed],
                              "rows_sha": hashlib.sha256(json.dumps(rows).encode()).hexdigest(),
                              "k": k, "max_n": max_n,
                              "out": [ngram.lookup(r, k, max_n) for r in rows]})
    # the reference's own literals and their neighbours
    for ctx, k, mn in [([1, 2, 3, 4, 1, 2], 2, 3), ([1, 2, 3, 1, 2], 5, 2), ([7, 8, 9, 1, 8, 5, 7, 8], 1, 2),
                       ([7, 8, 9, 1, 8, 5, 7, 8], 1, 1), ([1, 4, 2, 4, 3, 4], 1, 1), ([1, 2, 3], 3, 3),
                       ([5, 5, 5, 5], 4, 3), ([3], 2, 3), ([9, 9], 3, 3)]:
        cases.append({"rows": [ctx], "gen": None, "k": k, "max_n": mn, "out": [ngram.lookup(ctx, k, mn)]})
    return {"cases": cases}


def make_paged(kv) -> dict:
    from cache.paged import OutOfBlocks

    runs = []
    for seed, (bs, nb, n_ops) in enumerate([(3, 40, 250), (4, 16, 150), (16, 64, 150), (1, 24, 100)]):
        rng = random.Random(seed)
        cache = kv.KVCache(n_layers=1, n_kv_heads=1, head_dim=2, num_blocks=nb, block_size=bs,
                           dtype=torch.float32, device="cpu")
        live, next_id, ops_log = [], 0, []
        for _ in range(n_ops):
            r = rng.random()
            if r < 0.2 or not live:
                cache.add(next_id)
                live.append(next_id)
                op = ["add", next_id]
                next_id += 1
            elif r < 0.6:
                ids = rng.sample(live, min(len(live), rng.randint(1, 3)))
                n_new = [rng.randint(1, 2 * bs + 1) for _ in ids]
                try:
                    cache.append(ids, n_new)
                    op = ["append", ids, n_new, "ok"]
                except OutOfBlocks:
                    op = ["append", ids, n_new, "OutOfBlocks"]
            elif r < 0.85:
                s = rng.choice(live)
                length = rng.randint(0, cache.length(s))
                cache.truncate(s, length)
                op = ["truncate", s, length]
            else:
                s = live.pop(rng.randrange(len(live)))
                cache.free(s)
                op = ["free", s]
            st = cache.stats()
            ops_log.append({
                "op": op,
                "tables": {str(s): [t.blocks[:], t.length] for s, t in cache.tables.items()},
                "free": list(cache.allocator._free),
                "peak": cache.allocator.peak_used,
                "stats": [st.blocks_in_use, st.peak_blocks_in_use, st.slots_used],
            })
        runs.append({"block_size": bs, "num_blocks": nb, "seed": seed, "log": ops_log})
    return {"runs": runs}


def weights_sha(model) -> str:
    h = hashlib.sha256()
    for name, t in sorted(model.state_dict().items()):
        h.update(name.encode())
        h.update(t.detach().double().numpy().tobytes())
    return h.hexdigest()


def make_loop() -> dict:
    from conftest import early_exit_draft, new_cache, random_prompts  # reference tests/conftest.py
    from lm.load import tiny_model
    from spec.draft import ModelDraft
    from spec.loop import generate
    from spec.ngram import NGramDraft

    tiny = tiny_model(seed=0, dtype=torch.float64)
    draft_model = early_exit_draft(tiny)
    prompts = random_prompts(6, tiny.config.vocab_size, seed=4)
    runs = []
    for temperature, seed, kind in [(0.0, 0, "model"), (1.0, 7, "model"), (0.8, 11, "model"), (1.0, 3, "ngram")]:
        drafter = (ModelDraft(draft_model, new_cache(draft_model)) if kind == "model"
                   else NGramDraft(tiny.config.vocab_size))
        out, stats = generate(tiny, new_cache(tiny), drafter, prompts, 20, k=4, temperature=temperature,
                              generator=torch.Generator().manual_seed(seed))
        runs.append({"temperature": temperature, "seed": seed, "drafter": kind, "outputs": out,
                     "rounds": stats.rounds, "accepted": stats.accepted, "drafted": stats.drafted,
                     "attempts": stats.attempts, "accepts": stats.accepts,
                     "emitted_per_round": stats.emitted_per_round, "drafted_per_round": stats.drafted_per_round})
    return {"prompts": prompts, "weights_sha256": weights_sha(tiny), "max_new": 20, "k": 4, "runs": runs}


def main() -> None:
    accept, ngram, kv = ref_import()
    for name, fn in [("accept_gen.json", lambda: make_accept(accept)), ("ngram.json", lambda: make_ngram(ngram)),
                     ("paged_ops.json", lambda: make_paged(kv)), ("loop_tiny.json", make_loop)]:
        data = fn()
        (OUT / name).write_text(json.dumps(data, separators=(",", ":")))
        print(name, (OUT / name).stat().st_size, "bytes")


if __name__ == "__main__":
    main()
