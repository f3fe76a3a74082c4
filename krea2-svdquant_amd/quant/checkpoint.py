"""Writer of transformer-only SVDQuant checkpoints, with the SVD and quantization on any device.

Produces the directory that ``runtime.load.load_svdquant_transformer`` (and the reference
reader, ``runtime/load.py:52-132``) consumes, following the conversion recipe of reference
``scripts/convert_simulated.py:106-225``:

* targets are the ``nn.Linear`` modules under ``transformer_blocks.<i>.`` whose names end with
  a target suffix; the first / last ``skip_*_blocks`` blocks, ``attn.to_q`` / ``attn.to_k``
  with ``skip_qk``, layers without calibration statistics under ``require_calib`` and layers
  past ``max_layers`` are left dense;
* ranks: ``mlp_rank`` for ``ff`` layers, ``attn_rank`` for attention projections, ``rank``
  otherwise (``convert_simulated.py:96-101``);
* each layer: weight cast to bf16, SmoothQuant scale from the calibration absmax (identity
  without one), randomized rank-r SVD of ``W * s``, INT4 residual with fp16 group scales,
  stored as ``.qweight_packed`` / ``.weight_scales`` / ``.smooth_scale`` / ``.l1`` / ``.l2``
  (+ ``.bias``) under the ``.``->``__`` key, and a ``layers`` entry in the JSON;
* the JSON header fields (``format``, ``group_size``, ``calibrated``, ``num_blocks``,
  ``options`` ...) are those of ``convert_simulated.py:138-162``.

``svd_device="cuda"`` runs the decomposition and the quantization of each layer on the GPU
(one layer resident at a time); the stored tensors are always on the CPU.
"""
from __future__ import annotations

import argparse
import json
from pathlib import Path
from typing import Callable, Mapping

import torch
from safetensors.torch import save_file
from torch import nn

from ..config import SVDQuantConfig
from .convert import convert_linear

CONFIG_NAME = "svdquant_config.json"
TENSORS_NAME = "transformer_svdquant.safetensors"
FORMAT = "krea2-svdquant-transformer-v1"


def block_index(name: str) -> int | None:
    """``i`` of a ``transformer_blocks.<i>.…`` name, else None (``convert_simulated.py:87-93``)."""
    parts = name.split(".")
    if len(parts) >= 2 and parts[0] == "transformer_blocks" and parts[1].isdigit():
        return int(parts[1])
    return None


def rank_for(name: str, rank: int, attn_rank: int, mlp_rank: int) -> int:
    if ".ff." in name or name.endswith(("ff.gate", "ff.up", "ff.down")):
        return mlp_rank
    if ".attn." in name or ".to_" in name:
        return attn_rank
    return rank


def convert_transformer(transformer: nn.Module, out_dir: str | Path, *,
                        absmax: Mapping[str, torch.Tensor] | None = None, require_calib: bool = False,
                        base_model: str = "krea/Krea-2-Turbo", group_size: int | None = None,
                        rank: int | None = None, attn_rank: int | None = None, mlp_rank: int | None = None,
                        skip_first_blocks: int = 0, skip_last_blocks: int = 0, skip_qk: bool = False,
                        max_layers: int = 0, svd_oversample: int | None = None, svd_niter: int | None = None,
                        svd_device: str | torch.device | None = None, svd_exact: bool = False,
                        target_suffixes=None, seed: int | None = None,
                        log: Callable[[str], None] | None = print) -> dict:
    """Quantize the target linears of ``transformer`` into a checkpoint under ``out_dir``.

    ``absmax`` maps dotted layer names to the calibration ``max |x|`` per input channel (the
    reference's ``activation_absmax.pt``).  The model itself is not modified.  Returns the
    JSON metadata that was written.
    """
    from ..runtime.load import save_transformer_checkpoint_readme
    from ..runtime.replace import iter_named_linears

    cfg = SVDQuantConfig()
    group_size = cfg.weight_group_size if group_size is None else int(group_size)
    rank = cfg.default_rank if rank is None else int(rank)
    attn_rank = cfg.attn_rank if attn_rank is None else int(attn_rank)
    mlp_rank = cfg.mlp_rank if mlp_rank is None else int(mlp_rank)
    svd_oversample = cfg.svd_oversample if svd_oversample is None else int(svd_oversample)
    svd_niter = cfg.svd_niter if svd_niter is None else int(svd_niter)
    absmax = dict(absmax or {})
    if require_calib and not absmax:
        raise ValueError("require_calib needs calibration statistics (absmax)")
    say = log or (lambda _msg: None)
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)

    targets = [(n, m) for n, m in iter_named_linears(transformer, target_suffixes)
               if n.startswith("transformer_blocks.")]
    blocks = sorted({b for b in (block_index(n) for n, _ in targets) if b is not None})
    skipped_blocks = set(blocks[:skip_first_blocks])
    if skip_last_blocks:
        skipped_blocks |= set(blocks[len(blocks) - skip_last_blocks:])
    meta: dict = {
        "base_model": base_model,
        "format": FORMAT,
        "target_component": "transformer",
        "transformer_class": "Krea2Transformer2DModel",
        "runtime_target": "w4a16_plus_bf16_lowrank",
        "weight_bits": 4,
        "activation_bits": 16,
        "group_size": group_size,
        "calibrated": bool(absmax),
        "num_blocks": (blocks[-1] + 1) if blocks else 0,
        "options": {
            "rank": rank, "attn_rank": attn_rank, "mlp_rank": mlp_rank,
            "skip_first_blocks": skip_first_blocks, "skip_last_blocks": skip_last_blocks,
            "skip_qk": skip_qk, "max_layers": max_layers, "svd_oversample": svd_oversample,
            "svd_niter": svd_niter, "svd_exact": svd_exact,
        },
        "layers": {},
    }
    tensors: dict[str, torch.Tensor] = {}
    for name, mod in targets:
        if max_layers and len(meta["layers"]) >= max_layers:
            say(f"{len(meta['layers'])} layers written (max_layers); the remaining targets stay dense")
            break
        b = block_index(name)
        if b is not None and b in skipped_blocks:
            say(f"{name}: left dense (block {b} falls under skip_first_blocks / skip_last_blocks)")
            continue
        if skip_qk and name.endswith(("attn.to_q", "attn.to_k")):
            say(f"{name}: left dense (skip_qk)")
            continue
        calibrated = name in absmax
        if require_calib and not calibrated:
            say(f"{name}: left dense (require_calib, and no activation statistics for it)")
            continue
        r = rank_for(name, rank, attn_rank, mlp_rank)
        dev = torch.device(svd_device) if svd_device is not None else mod.weight.device
        w = mod.weight.detach().to(dev, torch.bfloat16)
        st = convert_linear(w, mod.bias, absmax[name].to(dev) if calibrated else None, rank=r,
                            group_size=group_size, oversample=svd_oversample, niter=svd_niter,
                            exact_svd=svd_exact, seed=seed)
        key = name.replace(".", "__")
        tensors[f"{key}.qweight_packed"] = st.qweight.cpu()
        tensors[f"{key}.weight_scales"] = st.weight_scales.cpu()
        tensors[f"{key}.smooth_scale"] = st.smooth_scale.cpu()
        tensors[f"{key}.l1"] = st.l1.cpu()
        tensors[f"{key}.l2"] = st.l2.cpu()
        if st.bias is not None:
            tensors[f"{key}.bias"] = st.bias.cpu()
        meta["layers"][name] = {"rank": r, "group_size": group_size, "shape": [int(v) for v in w.shape],
                                "calibrated": calibrated}
        say(f"{name}: {tuple(w.shape)} -> INT4 group {group_size} + rank {r}, "
            f"{'calibrated' if calibrated else 'uncalibrated'} smoothing")
    save_file(tensors, str(out / TENSORS_NAME))
    (out / CONFIG_NAME).write_text(json.dumps(meta, indent=2))
    save_transformer_checkpoint_readme(out, base_model)
    say(f"{len(meta['layers'])} quantized layers written to {out}")
    return meta


def main(argv=None) -> int:
    """Command line of the converter (the options of reference ``convert_simulated.py:18-84``).

    The base model is loaded with ``diffusers.Krea2Pipeline``, which must be installed
    together with a local copy of the weights; calibration statistics are read with
    ``torch.load(weights_only=True)``.
    """
    cfg = SVDQuantConfig()
    ap = argparse.ArgumentParser(description="Create a transformer-only SVDQuant checkpoint.")
    ap.add_argument("--model", default="krea/Krea-2-Turbo")
    ap.add_argument("--calib", default=None, help="directory holding activation_absmax.pt")
    ap.add_argument("--require-calib", action="store_true")
    ap.add_argument("--out", required=True)
    ap.add_argument("--group-size", type=int, default=cfg.weight_group_size)
    ap.add_argument("--rank", type=int, default=cfg.default_rank)
    ap.add_argument("--attn-rank", type=int, default=cfg.attn_rank)
    ap.add_argument("--mlp-rank", type=int, default=cfg.mlp_rank)
    ap.add_argument("--skip-first-blocks", type=int, default=0)
    ap.add_argument("--skip-last-blocks", type=int, default=0)
    ap.add_argument("--skip-qk", action="store_true")
    ap.add_argument("--max-layers", type=int, default=0)
    ap.add_argument("--svd-oversample", type=int, default=cfg.svd_oversample)
    ap.add_argument("--svd-niter", type=int, default=cfg.svd_niter)
    ap.add_argument("--svd-device", default=None, help="e.g. 'cuda' to decompose on the GPU")
    ap.add_argument("--svd-exact", action="store_true")
    args = ap.parse_args(argv)
    if args.require_calib and not args.calib:
        ap.error("--require-calib needs --calib")
    absmax = {}
    if args.calib:
        path = Path(args.calib) / "activation_absmax.pt"
        if not path.exists():
            ap.error(f"--calib given but {path} not found")
        absmax = torch.load(path, map_location="cpu", weights_only=True)
    try:
        from diffusers import Krea2Pipeline
    except Exception as exc:
        raise SystemExit(f"loading the base model needs diffusers with Krea2Pipeline: {exc}")
    transformer = Krea2Pipeline.from_pretrained(args.model, torch_dtype=torch.bfloat16).transformer.cpu()
    convert_transformer(transformer, args.out, absmax=absmax, require_calib=args.require_calib,
                        base_model=args.model, group_size=args.group_size, rank=args.rank,
                        attn_rank=args.attn_rank, mlp_rank=args.mlp_rank,
                        skip_first_blocks=args.skip_first_blocks, skip_last_blocks=args.skip_last_blocks,
                        skip_qk=args.skip_qk, max_layers=args.max_layers,
                        svd_oversample=args.svd_oversample, svd_niter=args.svd_niter,
                        svd_device=args.svd_device, svd_exact=args.svd_exact)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
