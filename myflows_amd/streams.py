"""The weight-gradient stream of a backward pass.

A batch-64 convolution product fills the GPU for one to two rounds of workgroups, and the last,
partial round leaves most CUs idle. Within ``Graph.backward`` each implicit convolution therefore
issues its dW (and conv-bias) product on a second HIP stream of default priority, ordered after
everything issued so far on the current stream, while its dX product, which the rest of the
backward pass waits for, stays on the current stream; the two grids run side by side. The current
stream is ordered after the second one once, when the pass ends (or earlier, when a gradient made
there is about to be added to on the current stream). Every product runs the same kernels with the
same plans as on one stream, so the gradients are the same bit for bit.

Memory. Everything the side stream reads or writes is allocated on the current stream and held by
the session until the join, so the caching allocator cannot hand a block out again before the side
stream's work on it is done: after the join, the current stream's later work is ordered after it.
Stream ordering is done inside the native library (an event recorded on one stream, waited for by
the other): the convolution's one call (``mfh_conv_backward_implicit_streams``) orders the side
stream after the main one and launches both products, and the join is one ``mfh_stream_wait``.
torch's ``wait_stream``, ``record_stream`` and stream switches would cost tens of microseconds of
host time per convolution, and the host issues a batch-64 step in about as long as the GPU runs it.
"""

from __future__ import annotations

import contextlib
import threading

import torch

from . import native

_local = threading.local()
_side_streams = {}


def side_stream(device_index):
    """The weight-gradient stream of a device (created once, default priority)."""
    stream = _side_streams.get(device_index)
    if stream is None:
        stream = torch.cuda.Stream(device=device_index)
        _side_streams[device_index] = stream
    return stream


class WeightGradSession:
    """The pair of streams of one backward pass, as raw handles."""

    def __init__(self):
        self.device = native.current_device_index()
        self.main = native._stream()
        self.side = side_stream(self.device).cuda_stream
        self.held = []  # tensors the side stream reads or writes, released at the join
        self.pending = False

    def usable(self):
        """Whether work can be forked now: the current stream is still the pass's main stream."""
        return native.current_device_index() == self.device and native._stream() == self.main

    def fork(self):
        """The side stream's handle and the list that receives the tensors of the work issued
        there; the caller's launch orders the side stream after the main stream itself
        (mfh_conv_backward_implicit_streams)."""
        self.pending = True
        return self.side, self.held

    def join(self):
        """Order the main stream after everything issued so far on the side stream, then release
        the held tensors."""
        if self.pending:
            native.stream_wait(self.main, self.side)
            self.pending = False
        self.held.clear()


def active():
    """The weight-gradient session of the running backward pass, or None."""
    return getattr(_local, "session", None)


@contextlib.contextmanager
def weight_grad_overlap(enabled=True):
    """Run the block as a backward pass whose weight gradients may take the side stream; the main
    stream (the current one on entry) is ordered after them on exit, also when the block raises."""
    if not enabled:
        yield None
        return
    previous = active()
    session = WeightGradSession()
    _local.session = session
    try:
        yield session
    finally:
        _local.session = previous
        session.join()
