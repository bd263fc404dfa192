"""A hipGraph of one decode step over fixed buffers, with the plan rebuilt at every replay.

Contract of src/sglang_decode/runtime/graph.py:6-79 (DecodeGraph(engine, keys,
kv_pairs), update / capture / replay, ValueError on the host for a step that does not
fit, outputs in the engine's reused buffers); the implementation is this module's.

The graph holds, per layer, a query buffer and a page table (paged) or a kv_indices
buffer of a fixed capacity (CSR); in CSR mode one kv_indptr buffer serves every layer,
since all layers of a step share the plan's lengths.  ``update`` validates the step on
the host, then stages lengths, split counts, the active count and (CSR) kv_indptr --
the exclusive prefix sum of the lengths, so it always agrees with them -- in pinned
host memory and uploads them with one asynchronous copy on the current stream, scatters
them into the plan, copies each layer's q and page table / kv_indices in, and marks the
inputs ready.  ``capture`` records ``engine.prepare()`` and every layer's
``engine.execute`` into one torch.cuda.CUDAGraph (a hipGraph on ROCm) after a few eager
warm-up steps on a side stream.  ``replay`` waits for the inputs and for the previous
replay, then launches the graph: the device plan is rebuilt from the staged lengths
every time.
"""
import torch

from .engine import DecodeEngine


class DecodeGraph:
    def __init__(self, engine: DecodeEngine, keys, kv_pairs, index_capacity=None):
        """``keys``: one PlanKey per layer, all equal (the layers share one plan).
        ``kv_pairs``: (k, v) per layer.  ``index_capacity``: CSR mode, the kv_indices
        entries each layer's buffer holds (one int per layer); None for paged KV."""
        n_layers = len(engine.layers)
        if len(keys) != n_layers or len(kv_pairs) != n_layers:
            raise ValueError(f"DecodeGraph: the engine has {n_layers} layers, got {len(keys)} plan keys and "
                             f"{len(kv_pairs)} KV pairs")
        if n_layers == 0 or len(set(keys)) != 1:
            raise ValueError("DecodeGraph: every layer must carry the same plan key (layers with different "
                             "keys need plans, and graphs, of their own)")
        self.engine, self.kv_pairs = engine, list(kv_pairs)
        c, dev = engine.config, engine.plan.device
        bcap = c.batch_capacity
        self.csr = index_capacity is not None
        self.q = [torch.empty_like(layer.output) for layer in engine.layers]
        # [lengths | splits | active | kv_indptr]: one upload per update
        self._meta = torch.zeros(3 * bcap + 2, dtype=torch.int32, device=dev)
        self._meta_host = torch.zeros(3 * bcap + 2, dtype=torch.int32, pin_memory=dev.type == "cuda")
        if self.csr:
            if len(index_capacity) != n_layers:
                raise ValueError(f"DecodeGraph: {n_layers} layers need {n_layers} kv_indices capacities")
            self.pages = [torch.zeros(int(n), dtype=torch.int32, device=dev) for n in index_capacity]
            self.indptr = [self._meta[2 * bcap + 1:]] * n_layers
        else:
            self.pages = [torch.zeros((bcap, c.max_pages), dtype=torch.int32, device=dev) for _ in keys]
            self.indptr = [None] * n_layers
        self.ready, self.done, self._staged = torch.cuda.Event(), torch.cuda.Event(), torch.cuda.Event()
        self.graph = None
        self._updated = self._replayed = self._staging = False

    def _check_step(self, queries, page_tables, lengths, splits):
        c = self.engine.config
        n = len(lengths)
        if not 1 <= n <= c.batch_capacity:
            raise ValueError(f"DecodeGraph.update: batch {n} outside [1, {c.batch_capacity}]; use a graph with a "
                             "larger capacity (or the upstream path)")
        if len(splits) != n:
            raise ValueError(f"DecodeGraph.update: {n} lengths but {len(splits)} split counts")
        if min(lengths) < 0 or max(lengths) > c.max_context:
            raise ValueError(f"DecodeGraph.update: a context length is outside [0, {c.max_context}]")
        if min(splits) < 1 or max(splits) > c.max_splits:
            raise ValueError(f"DecodeGraph.update: a split count is outside [1, {c.max_splits}]")
        if len(queries) != len(self.q) or len(page_tables) != len(self.pages):
            raise ValueError(f"DecodeGraph.update: {len(self.q)} layers, got {len(queries)} query tensors and "
                             f"{len(page_tables)} page tables")
        total = sum(int(x) for x in lengths)
        for i, (q, table) in enumerate(zip(queries, page_tables)):
            if tuple(q.shape) != (n, c.query_heads, c.head_dim):
                raise ValueError(f"DecodeGraph.update: layer {i} q is {tuple(q.shape)}, expected "
                                 f"{(n, c.query_heads, c.head_dim)}")
            if self.csr:
                if table.dim() != 1 or not total <= table.numel() <= self.pages[i].numel():
                    raise ValueError(f"DecodeGraph.update: layer {i} kv_indices has {table.numel()} entries; the "
                                     f"step needs {total} and the graph holds {self.pages[i].numel()}")
            elif tuple(table.shape) != (n, c.max_pages):
                raise ValueError(f"DecodeGraph.update: layer {i} page table is {tuple(table.shape)}, expected "
                                 f"{(n, c.max_pages)}")

    def update(self, queries, page_tables, lengths, splits):
        """Stage one step's inputs: host-known lengths and split counts (no device readback),
        per-layer q [n, Hq, D] and page table [n, max_pages] or (CSR) kv_indices holding the
        rows of request r at [sum of the earlier lengths, + L_r)."""
        lengths, splits = [int(x) for x in lengths], [int(x) for x in splits]
        self._check_step(queries, page_tables, lengths, splits)
        c, p = self.engine.config, self.engine.plan
        bcap, n = c.batch_capacity, len(lengths)
        stream = torch.cuda.current_stream(p.device)
        if self._replayed:
            stream.wait_event(self.done)  # the last replay still reads the buffers below
        if self._staging:
            self._staged.synchronize()    # the last upload has left the pinned buffer
        host = self._meta_host
        host.zero_()
        host[:n] = torch.tensor(lengths, dtype=torch.int32)
        host[bcap:2 * bcap] = 1
        host[bcap:bcap + n] = torch.tensor(splits, dtype=torch.int32)
        host[2 * bcap] = n
        host[2 * bcap + 2:2 * bcap + 2 + n] = torch.cumsum(torch.tensor(lengths, dtype=torch.int64), 0)
        self._meta.copy_(host, non_blocking=True)
        self._staged.record(stream)
        self._staging = True
        p.lengths.copy_(self._meta[:bcap])
        p.splits.copy_(self._meta[bcap:2 * bcap])
        p.active.copy_(self._meta[2 * bcap:2 * bcap + 1])
        for dst_q, dst_t, q, table in zip(self.q, self.pages, queries, page_tables):
            dst_q[:n].copy_(q)
            dst_t[:table.shape[0]].copy_(table)
        self.ready.record(stream)
        self._updated = True

    def _step(self):
        self.engine.prepare()
        for layer, (k, v) in enumerate(self.kv_pairs):
            self.engine.execute(self.q[layer], k, v, self.pages[layer], layer=layer, indptr=self.indptr[layer])

    def capture(self, warmup=3):
        """Record the step (plan build + every layer) into the graph; a GPU operation the
        caller opts into after a representative update()."""
        if self.graph is not None:
            raise RuntimeError("DecodeGraph.capture: already captured; a different geometry needs a new DecodeGraph")
        if not self._updated:
            raise RuntimeError("DecodeGraph.capture: update() the graph with representative inputs first")
        side = torch.cuda.Stream(device=self.engine.plan.device)
        side.wait_event(self.ready)
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self._step()
        side.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            self._step()
        self.graph = graph
        self.done.record(side)
        self._replayed = True

    def replay(self):
        """Launch the captured step on the current stream; returns the layers' output buffers."""
        if self.graph is None:
            raise RuntimeError("DecodeGraph.replay: nothing captured (update() with representative inputs, "
                               "then capture())")
        stream = torch.cuda.current_stream(self.engine.plan.device)
        stream.wait_event(self.ready)
        if self._replayed:
            stream.wait_event(self.done)
        self.graph.replay()
        self.done.record(stream)
        self._replayed = True
        return [layer.output for layer in self.engine.layers]
