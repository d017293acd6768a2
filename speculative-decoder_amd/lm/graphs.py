"""HIP-graph replay of the fixed-shape forwards of the round loop.

A speculative round runs the same few shapes again and again: the verify
pass (B rows of k+1 tokens, ending in the output head fused with the
softmax / one-hot) and the k draft steps (B rows of 1 token, ending in the
same fused head, then the inverse-CDF sampler at T > 0, each step's token
feeding the next step).  Each is captured once per
(cache, batch, width, temperature, context bucket) and replayed; block
allocation and the per-step metadata stay on the host side of the replay
(one block-plan launch and one small copy per round), because they decide
*which* slots the captured kernels touch, not *what* they compute.

Every captured kernel reads row metadata, block tables, RoPE tables and its
own attention workspace through fixed device pointers.  A graph is captured
for a context bucket (the attention grid covers `bucket` keys; rows shorter
than that exit early) and is recaptured if the cache's table storage or the
RoPE tables were reallocated since.

Set SPECDEC_GRAPHS=0 to run the same kernels eagerly.
"""
from __future__ import annotations

import gc
import os
import weakref

import torch

from cache.kv import KVCache
from lm.forward import forward_core
from lm.model import Llama
from specdec import ops

# Context buckets of 2048 keys: up to four 512-token splits, which the
# attention kernel folds inside one workgroup (no combine launch).
BUCKET = 2048


def enabled() -> bool:
    return os.environ.get("SPECDEC_GRAPHS", "1") != "0"


def bucket_for(max_total: int) -> int:
    return -(-max_total // BUCKET) * BUCKET


def _capture(run):
    """Warm `run` up on a side stream, then capture it; returns (graph, outputs).

    The garbage collector is run first and kept off until the capture ends:
    a collection inside a capture could destroy another graph (and release
    its memory pool), which HIP does not allow while a stream is capturing."""
    gc.collect()
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            run()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            outs = run()
    finally:
        if was_enabled:
            gc.enable()
    return graph, outs


class _Captured:
    def __init__(self, llama: Llama, cache: KVCache, batch: int, bucket: int, width: int,
                 latency: bool = False) -> None:
        # the cache owns its runners (cache.graphs); a weak reference back keeps
        # that from being a cycle, so dropping a cache frees its graphs at once
        self._cache = weakref.ref(cache)
        self.llama, self.batch, self.bucket = llama, batch, bucket
        dev = cache.device
        self.ws = ops.AttentionWorkspace(dev)
        ops.head_workspace(dev)  # allocated (and zeroed) once, outside any capture
        cfg = llama.config
        self.split = (ops.latency_split(batch, width, cfg.num_attention_heads, cfg.num_key_value_heads, bucket)
                      if latency else 0)
        self.ws.reserve(ops.attention_workspace_floats(batch, width, cfg.num_attention_heads, cfg.num_key_value_heads,
                                                       cfg.head_dim, bucket, self.split))
        self.graph = None
        self.outs = None
        self._ptrs = None

    @property
    def cache(self) -> KVCache:
        cache = self._cache()
        if cache is None:
            raise RuntimeError("the cache of this graph runner no longer exists")
        return cache

    def _pointers(self):
        return (self.cache.table_tensor.data_ptr(), self.llama.rope_cos.data_ptr(), self.llama.rope_sin.data_ptr())

    def replay(self, prepare, run):
        """prepare() writes the static inputs; run() is the captured work."""
        prepare()
        if self.graph is None or self._pointers() != self._ptrs:
            self.graph = None
            self.graph, self.outs = _capture(run)
            self._ptrs = self._pointers()
            prepare()  # the warm-up may have advanced chained inputs
        self.graph.replay()
        return self.outs


class VerifyGraph(_Captured):
    """forward over [B, width] (every row `width` new tokens) + probabilities."""

    def __init__(self, llama, cache, batch, width, temperature, bucket):
        super().__init__(llama, cache, batch, bucket, width)
        dev = cache.device
        self.temperature = temperature
        self.ids = torch.zeros(batch, width, dtype=torch.int64, device=dev)
        self.meta = torch.zeros(3, batch, dtype=torch.int32, device=dev)

    def run(self, ids: torch.Tensor, meta: torch.Tensor) -> torch.Tensor:
        def prepare():
            self.ids.copy_(ids, non_blocking=True)
            self.meta.copy_(meta, non_blocking=True)

        def work():
            return forward_core(self.llama, self.cache, self.meta, self.ids, self.bucket, None, self.ws,
                                temperature=self.temperature)

        return self.replay(prepare, work)


class DraftStepGraph(_Captured):
    """One draft step over right-padded [B, width] ids: forward of each row's
    last real token, probabilities, and an inverse-CDF sample with u[B]."""

    def __init__(self, llama, cache, batch, width, temperature, bucket, latency=True):
        super().__init__(llama, cache, batch, bucket, width, latency=latency)
        dev = cache.device
        self.temperature = temperature
        self.ids = torch.zeros(batch, width, dtype=torch.int64, device=dev)
        self.meta = torch.zeros(3, batch, dtype=torch.int32, device=dev)
        self.u = torch.zeros(batch, dtype=torch.float32, device=dev)
        self.token = torch.zeros(batch, dtype=torch.int64, device=dev)
        # one token per row (the usual first step): each row's last token is
        # position 0, so no launch computes it
        self.last0 = torch.zeros(batch, dtype=torch.int64, device=dev) if width == 1 else None

    def run(self, ids, meta, u):
        def prepare():
            self.ids.copy_(ids, non_blocking=True)
            self.meta.copy_(meta, non_blocking=True)
            self.u.copy_(u, non_blocking=True)

        def work():
            last = self.last0 if self.last0 is not None else self.meta[2].long() - 1
            if self.temperature == 0.0:  # the one-hot row's inverse-CDF draw is its argmax
                q = forward_core(self.llama, self.cache, self.meta, self.ids, self.bucket, last, self.ws, self.split,
                                 temperature=0.0, index_out=self.token)
                return q, self.token
            q = forward_core(self.llama, self.cache, self.meta, self.ids, self.bucket, last, self.ws, self.split,
                             temperature=self.temperature)
            return q, ops.sample_inverse_cdf(q, self.u)

        return self.replay(prepare, work)


class DraftChainGraph(_Captured):
    """`steps` consecutive one-token draft steps, each sampled token feeding
    the next step on the device.  Outputs q [B, steps, V] and tokens [B, steps]."""

    def __init__(self, llama, cache, batch, steps, temperature, bucket, latency=True):
        super().__init__(llama, cache, batch, bucket, 1, latency=latency)
        dev = cache.device
        self.temperature, self.steps = temperature, steps
        v = llama.config.vocab_size
        self.first = torch.zeros(batch, 1, dtype=torch.int64, device=dev)
        self.metas = torch.zeros(steps, 3, batch, dtype=torch.int32, device=dev)
        self.u = torch.zeros(steps, batch, dtype=torch.float32, device=dev)
        self.q = torch.zeros(batch, steps, v, dtype=torch.float32, device=dev)
        self.tokens = torch.zeros(batch, steps, dtype=torch.int64, device=dev)

    def run(self, first, metas, u):
        def prepare():
            self.first.copy_(first.view(-1, 1), non_blocking=True)
            self.metas.copy_(metas, non_blocking=True)
            self.u.copy_(u, non_blocking=True)

        def work():
            ids = self.first
            for i in range(self.steps):
                if self.temperature == 0.0:
                    # the inverse-CDF draw from a one-hot row is its argmax for
                    # every u, so the head writes the token itself
                    forward_core(self.llama, self.cache, self.metas[i], ids, self.bucket, None, self.ws, self.split,
                                 temperature=0.0, out=self.q[:, i], index_out=self.tokens[:, i])
                else:
                    forward_core(self.llama, self.cache, self.metas[i], ids, self.bucket, None, self.ws, self.split,
                                 temperature=self.temperature, out=self.q[:, i])
                    self.tokens[:, i].copy_(ops.sample_inverse_cdf(self.q[:, i], self.u[i]))
                ids = self.tokens[:, i:i + 1]
            return self.q, self.tokens

        return self.replay(prepare, work)


def get(cache: KVCache, kind, llama: Llama, *key):
    """The cached graph runner of `kind` for this cache and key, created on
    first use (capture happens at its first run)."""
    full = (kind.__name__, id(llama)) + key
    runner = cache.graphs.get(full)
    if runner is None:
        runner = cache.graphs[full] = kind(llama, cache, *key)
    return runner
