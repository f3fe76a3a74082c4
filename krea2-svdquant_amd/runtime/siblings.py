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

``run_grouped`` goes further for W4A4 layers: one activation pass per layer (each has its own
smoothing vector, so the codes differ), then the layers' GEMMs in ONE launch
(``svdq_w4a4_gemm_siblings``), whose workgroups take the layers' output tiles back to back.  At
M = 4352 the four attention inputs then run 2040 tiles in 8 rounds over the 256 CUs instead of
3.19 + 0.8 + 0.8 + 3.19 rounds rounded up to 10, and ff.gate + ff.up 4352 tiles in 17 rounds
instead of 18.  The tiles are the single-layer kernel's, so the outputs are again bit-identical.
W4A16 layers take the same route (``svdq_w4a16_gemm_siblings``): each layer's x_hat pass, then
one launch of the specialized-wave kernel's 192 x 256 tiles where its rounds cost no more than
the layers' own launches: the attention inputs at M = 2304 run 720 tiles in 3 rounds (383 us)
instead of 538 us in four launches.
"""
from __future__ import annotations

from typing import Callable, Sequence

import torch
from torch import Tensor, nn

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


def _groupable(x: Tensor, layers: Sequence[nn.Module]) -> bool:
    from ..kernels.hip.backend import FAST_GROUPS
    from ..kernels.hip.lib import SVDQ_MAX_SIBLINGS
    from .linear import SVDQuantLinear
    if not x.is_cuda or not 2 <= len(layers) <= SVDQ_MAX_SIBLINGS:
        return False
    if not all(isinstance(m, SVDQuantLinear) for m in layers):
        return False
    l0 = layers[0]
    mode = l0._mode(x.device)
    return all(m._mode(x.device) == mode and m.group_size in FAST_GROUPS and m.group_size == l0.group_size
               and m.original_shape[1] == l0.original_shape[1] and m.padded_in_features == l0.padded_in_features
               for m in layers)


def run_grouped(x: Tensor, layers: Sequence[nn.Module]) -> list[Tensor]:
    """``[layer(x) for layer in layers]``; when every layer is an ``SVDQuantLinear`` of one mode
    (W4A4 or W4A16) with group size 64 or 128 and the same in_features (2 to 4 layers, on the
    GPU), their GEMMs run as one launch (``forward_prepared_siblings``; W4A16 where the grouped
    tiles pay), each with its layer's LoRA adapters.  Other layer sets run one after another."""
    if not _groupable(x, layers):
        return [m(x) for m in layers]
    from ..kernels.hip.backend import forward_prepared_siblings
    preps = [m._prepare(x.device, with_adapters=bool(m.lora_adapters)) for m in layers]
    return forward_prepared_siblings(x, preps, mode=layers[0]._mode(x.device))
