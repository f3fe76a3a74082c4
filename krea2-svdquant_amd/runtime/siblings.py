"""Sibling linears: several layers applied to the same input, issued concurrently on one GPU.

A Krea-2 block feeds one normed activation tensor to four quantized linears (``attn.to_q``,
``to_k``, ``to_v``, ``to_gate``) and another to two (``ff.gate``, ``ff.up``).  The reference runs
them one after another, each through ``SVDQuantLinear.forward``
(``src/krea2_svdquant/runtime/linear.py:156``; diffusers' block calls the modules in turn), and so does
``SVDQuantLinear`` here unless the caller groups them with ``run_concurrent``.

Alone, each layer leaves CUs idle at its end: its W4A4 GEMM cuts the output into 256 x 128 tiles,
one workgroup per CU at a time, so at M = 4352 to_q (17 x 48 = 816 tiles) runs 3.19 rounds over
the 256 CUs and to_k / to_v (204 tiles) fill less than one round; the activation passes before
them are short, latency-bound launches.  ``run_concurrent`` issues the first layer on the caller's
stream and every other one on a side stream of the same device (default priority), so the
hardware queues hand idle CUs the siblings' workgroups.  The kernels, their arguments and the
per-call buffers are the same as in sequential calls (the library keeps no state between calls:
every buffer is allocated per call on the current stream), so the outputs are bit-identical.

Ordering: every side stream first waits for the caller's stream (the input is ready); the caller's
stream then waits for every side stream, and each output made on a side stream is recorded as
used on the caller's stream, so the caching allocator cannot hand its memory to later work of the
side stream while the caller still reads it.
"""
from __future__ import annotations

from typing import Callable, Sequence

import torch
from torch import Tensor

_SIDE_STREAMS: dict[int, list] = {}


def side_streams(device: torch.device, n: int) -> list:
    """``n`` side streams of ``device``, created once per process and device, default priority."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    pool = _SIDE_STREAMS.setdefault(index, [])
    while len(pool) < n:
        pool.append(torch.cuda.Stream(device=index))
    return pool[:n]


def run_concurrent(x: Tensor, fns: Sequence[Callable[[Tensor], Tensor]]) -> list[Tensor]:
    """``[f(x) for f in fns]``, with the calls issued concurrently when ``x`` is on a GPU.

    ``fns[0]`` runs on the current stream, the others on side streams; on return the current
    stream is ordered after all of them.  Off the GPU (or with one function) the calls run in
    order on the host.  Put the longest layer first: it starts first."""
    if not x.is_cuda or len(fns) < 2:
        return [f(x) for f in fns]
    main = torch.cuda.current_stream(x.device)
    side = side_streams(x.device, len(fns) - 1)
    for s in side:
        s.wait_stream(main)
    outs = [fns[0](x)]
    for f, s in zip(fns[1:], side):
        with torch.cuda.stream(s):
            outs.append(f(x))
    for y, s in zip(outs[1:], side):
        main.wait_stream(s)
        y.record_stream(main)
    return outs
