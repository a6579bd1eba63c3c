"""A training step's forward and backward pass recorded once as a HIP graph and replayed.

A batch-64 ResNet18 step issues about two hundred kernel launches, stream orderings and ctypes
calls, and the Python host needs about as long to issue them as the GPU needs to run them: the
step is then bound by the host, and faster kernels do not shorten it. ``CapturedStep`` runs
``Graph.forward`` and ``Graph.backward`` once under HIP stream capture (``torch.cuda.CUDAGraph``,
which is hipGraph on ROCm) and afterwards replays the recorded graph with one launch per step. The
recorded work is exactly the eager pass's: the same kernels with the same plans on the same
buffers, the dW products on the weight-gradient stream joined into the capture by the same event
orderings, so every replay gives the eager step's bits.

What a replay keeps fixed is what the recording saw:

* the shapes, dtypes and devices of every input, and which leaves need gradients;
* the tensors: node values, gradients and the library's workspaces live in the graph's private
  memory pool, so the inputs must be refreshed in place (``Variable.value.copy_``) and the outputs
  (``node.value``, the parameter gradients) are overwritten by the next replay;
* the parameters are read through their tensors, so in-place optimiser updates between replays
  (``Adam.update``) are seen by the next replay.

The optimiser update itself stays eager: Adam's bias corrections are host scalars of the step
count. Nothing in the recorded pass may synchronise with the host or allocate outside torch's
caching allocator; the library itself never allocates and writes no memset nodes.
"""

from __future__ import annotations

import torch

from .graph import Graph


class _ReplayedStep:
    """The optimiser side of a replayed step: the recorded gradient buffers of the trainable leaves
    (refreshed by every replay) go to ``acc_gradient`` as the eager ``one_step`` would put them."""

    def __init__(self, optimizer):
        self.optimizer = optimizer
        graph = optimizer.graph
        if not isinstance(graph, Graph):
            raise TypeError(f"{type(self).__name__} needs an optimiser over a Graph")
        device = graph.target_node.value.device if graph.target_node.value is not None else None
        if not torch.cuda.is_available() or (device is not None and device.type != "cuda"):
            raise RuntimeError(f"{type(self).__name__} records HIP work and needs the graph on a GPU")
        self.replays = 0

    def _keep_gradients(self):
        graph = self.optimizer.graph
        self.gradients = {node: node.grad for node in graph.nodes if node.trainable is True and node.grad is not None}

    def forward_backward(self):
        raise NotImplementedError

    def one_step(self):
        """The optimiser's ``one_step``: replay, then add the gradients into ``acc_gradient``.

        The first step after an update hands the recorded buffers themselves to the optimiser; a
        further accumulation step first gives those entries buffers of their own, since the replay
        overwrites the recorded ones."""
        opt = self.optimizer
        if opt.acc_no > 0:
            for node, held in list(opt.acc_gradient.items()):
                if held is self.gradients.get(node):
                    opt.acc_gradient[node] = held.clone()
        self.forward_backward()
        for node, gradient in self.gradients.items():
            held = opt.acc_gradient.get(node)
            if held is None:
                opt.acc_gradient[node] = gradient
            else:
                held += gradient
        opt.acc_no += 1

    def update(self):
        self.optimizer.update()


class CapturedStep(_ReplayedStep):
    """``one_step()`` of an optimiser (forward, backward and gradient accumulation) as one HIP graph
    replay. ``warmup`` eager passes run first (on a side stream, as stream capture requires), so
    that plans, weight orders and workspaces exist before the recording."""

    def __init__(self, optimizer, warmup=2):
        super().__init__(optimizer)
        graph = optimizer.graph
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(max(1, int(warmup))):
                graph.forward()
                graph.backward()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.hip_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.hip_graph):
            graph.forward()
            graph.backward()
        self._keep_gradients()

    def forward_backward(self):
        """Replay the recorded forward and backward pass (the outputs and gradients are updated in
        place)."""
        self.hip_graph.replay()
        self.replays += 1


class RecordedStep(_ReplayedStep):
    """``one_step()`` of an optimiser as a libmfhip program: one ctypes call that issues the
    forward and backward pass's kernel launches and stream orderings again, from C, as the eager
    pass issued them (on the same streams, so the weight-gradient stream still runs beside the dX
    products).

    ``warmup`` eager passes run first, so that plans, weight orders and workspaces exist; then one
    more eager pass runs while the library records it (mfh_program_begin / mfh_program_end), with
    every tensor it allocates in a private memory pool: the blocks of the pass's temporaries stay
    reserved for the replays, which write them in the recorded order. Every GPU write of the pass
    is a library launch (the backward's seed too), so the program is the whole pass. The same rules
    as for ``CapturedStep`` hold: fixed shapes and leaf flags, inputs refreshed in place, outputs and
    gradients overwritten by each replay, the optimiser update eager."""

    def __init__(self, optimizer, warmup=2):
        from . import native
        super().__init__(optimizer)
        graph = optimizer.graph
        for _ in range(max(0, int(warmup))):
            graph.forward()
            graph.backward()
        self.pool = torch.cuda.MemPool()
        self.program = None
        with torch.cuda.use_mem_pool(self.pool):
            native.program_begin()
            try:
                graph.forward()
                graph.backward()
            finally:
                self.program, self.launches = native.program_end()
        self._native = native
        self._keep_gradients()

    def forward_backward(self):
        """Issue the recorded forward and backward pass again (outputs and gradients in place)."""
        self._native.program_run(self.program)
        self.replays += 1

    def close(self):
        if self.program:
            self._native.program_free(self.program)
            self.program = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
