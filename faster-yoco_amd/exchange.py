"""The owner's BF16 exchange after the step, pipelined with the Adam launches.

The reference all-gathers every owner's BF16 segment into the flat parameter buffer once the whole step is done
(``dist.all_gather_into_tensor``, yoco/tasks/zero1_fast.py:224-226).  Here the step runs as one Adam launch per range
of table rows (``z1_adam_cast_rows``, the same results as one launch), and each finished range is handed to a sender
on a second stream as soon as its launch completes, so the exchange of the first ranges overlaps the update of the
last ones.  Only the sending side exists on one GPU: ``send(first, last)`` is the caller's (a peer copy or a
collective on the side stream in a multi-GPU job; in the tests and the bench, a copy into a local buffer laid out as
a peer's flat buffer).
"""
import torch

__all__ = ['even_pieces', 'PipelinedExchange']


def even_pieces(numels, k):
    """Row boundaries [0, ..., len(numels)] splitting the rows into at most k ranges of about equal element counts
    (each range ends at the first row that reaches its share)."""
    total = sum(int(n) for n in numels)
    k = max(1, min(int(k), len(numels)))
    bounds, acc, want = [0], 0, 1
    for i, n in enumerate(numels):
        acc += int(n)
        if want < k and acc * k >= want * total and i + 1 < len(numels):
            bounds.append(i + 1)
            want += 1
    bounds.append(len(numels))
    return bounds


class PipelinedExchange:
    """step(opt): opt.step() in row ranges of its FlatShard; after each range, an event on the current stream, the
    side stream waits for it and calls send(first, last) with the range's [first, last) positions in the flat
    buffers.  At the end the current stream waits for the side stream, so later work (the next step's Adam writes the
    same BF16 rows) is ordered after the sends."""

    def __init__(self, shard, pieces, send, stream=None):
        self.shard = shard
        self.pieces = list(pieces)
        self.send = send
        self.stream = stream if stream is not None else torch.cuda.Stream(device=shard.device)   # default priority

    def step(self, opt):
        if opt.shard is not self.shard:
            raise RuntimeError('exchange: the optimizer updates another shard')
        cur = torch.cuda.current_stream(self.shard.device)

        def on_piece(a, b):
            ev = torch.cuda.Event()
            ev.record(cur)
            self.stream.wait_event(ev)
            first, last = self.shard.row_elements(a, b)
            with torch.cuda.stream(self.stream):
                self.send(first, last)

        opt.step(pieces=self.pieces, on_piece=on_piece)
        cur.wait_stream(self.stream)
