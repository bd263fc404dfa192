"""Standalone hipGraph owner: stable pointers, replayed plan, layer-private scratch.

Same lifecycle as src/sglang_decode/runtime/graph.py:6-79.  ``update()`` checks
capacity on the host (ValueError), waits for the previous replay, copies lengths,
splits, active, per-layer q and page tables into fixed buffers and records
``ready``.  ``capture()`` warms up on a side stream and captures ``prepare`` plus
every layer's ``execute`` into one graph (torch.cuda.CUDAGraph is a hipGraph on
ROCm), so the plan is rebuilt on the device at every ``replay()``.
"""
import torch

from .engine import DecodeEngine


class DecodeGraph:
    def __init__(self, engine: DecodeEngine, keys, kv_pairs, indptrs=None):
        if len(keys) != len(engine.layers) or len(kv_pairs) != len(keys):
            raise ValueError("one key and KV pair per layer required")
        if not keys or any(key != keys[0] for key in keys):
            raise ValueError("incompatible layers require separate plan/graph instances")
        self.engine, self.kv_pairs = engine, kv_pairs
        c, p = engine.config, engine.plan
        self.csr = indptrs is not None
        self.q = [torch.empty_like(layer.output) for layer in engine.layers]
        if self.csr:
            # CSR: per-layer kv_indptr [Bcap+1] and kv_indices sized by the caller's pool.
            if len(indptrs) != len(keys):
                raise ValueError("one kv_indptr/kv_indices pair per layer required")
            self.indptr = [torch.zeros(c.batch_capacity + 1, dtype=torch.int32, device=p.device)
                           for _ in keys]
            self.pages = [torch.zeros(int(cap), dtype=torch.int32, device=p.device)
                          for cap in indptrs]
        else:
            self.indptr = [None] * len(keys)
            self.pages = [torch.zeros((c.batch_capacity, c.max_pages), dtype=torch.int32,
                                      device=p.device) for _ in keys]
        self.ready, self.done = torch.cuda.Event(), torch.cuda.Event()
        self.graph = None
        self.has_run = False

    def update(self, queries, page_tables, lengths, splits, indptrs=None):
        """Host lengths are already known by the scheduler; no device scalar readback."""
        c, p = self.engine.config, self.engine.plan
        if not 0 < len(lengths) <= c.batch_capacity or len(splits) != len(lengths):
            raise ValueError("choose a larger graph or upstream before submitting")
        if any(x < 0 or x > c.max_context for x in lengths):
            raise ValueError("context outside graph capacity")
        if any(x < 1 or x > c.max_splits for x in splits):
            raise ValueError("split capacity exceeded")
        if len(queries) != len(self.q) or len(page_tables) != len(self.pages):
            raise ValueError("layer count mismatch")
        n = len(lengths)
        for q, pages in zip(queries, page_tables):
            if tuple(q.shape) != (n, c.query_heads, c.head_dim):
                raise ValueError("input shape mismatch")
            if not self.csr and tuple(pages.shape) != (n, c.max_pages):
                raise ValueError("input shape mismatch")
            if self.csr and pages.numel() > self.pages[0].numel():
                raise ValueError("kv_indices exceed the captured index capacity")
        if self.csr and (indptrs is None or len(indptrs) != len(self.indptr)):
            raise ValueError("CSR graphs need one kv_indptr per layer")
        stream = torch.cuda.current_stream(p.device)
        if self.has_run:
            stream.wait_event(self.done)
        host_l = torch.zeros(c.batch_capacity, dtype=torch.int32)
        host_s = torch.ones(c.batch_capacity, dtype=torch.int32)
        host_l[:n] = torch.tensor(lengths, dtype=torch.int32)
        host_s[:n] = torch.tensor(splits, dtype=torch.int32)
        p.lengths.copy_(host_l)
        p.splits.copy_(host_s)
        p.active.fill_(n)
        for i, (q, pages) in enumerate(zip(queries, page_tables)):
            self.q[i][:n].copy_(q)
            self.pages[i][:pages.shape[0]].copy_(pages)
            if self.csr:
                self.indptr[i][:n + 1].copy_(indptrs[i][:n + 1])
        self.ready.record(stream)

    def _step(self):
        self.engine.prepare()
        for i, (k, v) in enumerate(self.kv_pairs):
            self.engine.execute(self.q[i], k, v, self.pages[i], layer=i, indptr=self.indptr[i])

    def capture(self, warmup=3):
        """Explicit opt-in GPU operation.  Never invoked at import."""
        if self.graph is not None:
            raise RuntimeError("capture once; create another instance to change geometry")
        stream = torch.cuda.Stream(device=self.engine.plan.device)
        stream.wait_event(self.ready)
        with torch.cuda.stream(stream):
            for _ in range(warmup):
                self._step()
        stream.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=stream):
            self._step()
        self.done.record(stream)
        self.has_run = True

    def replay(self):
        if self.graph is None:
            raise RuntimeError("capture after initializing representative inputs")
        stream = torch.cuda.current_stream(self.engine.plan.device)
        stream.wait_event(self.ready)
        if self.has_run:
            stream.wait_event(self.done)
        self.graph.replay()
        self.done.record(stream)
        self.has_run = True
        return [layer.output for layer in self.engine.layers]
