"""Reader for transformer-only SVDQuant checkpoints: swaps quantized linears into a model.

Mirror of reference ``src/krea2_svdquant/runtime/load.py``.  The checkpoint is a directory with

* ``svdquant_config.json`` -- ``{"group_size": G, "layers": {dotted_name: {"rank", "group_size",
  "shape": [N, K], "calibrated"}}, ...}`` (written by reference
  ``scripts/convert_simulated.py:138-162,209-214`` and by ``quant.checkpoint`` here);
* ``transformer_svdquant.safetensors`` -- per layer, under the key ``dotted_name`` with ``.``
  replaced by ``__`` (``load.py:16-17``): ``.qweight_packed`` uint8 [N, Kp/2],
  ``.weight_scales`` fp16 [N, Kp/G], ``.smooth_scale`` bf16 [K], ``.l1`` bf16 [N, r],
  ``.l2`` bf16 [r, K] and, when the dense layer had one, ``.bias`` bf16 [N].

``load_svdquant_transformer`` keeps the reference signature and return value (the config dict
with a ``_load_report``) and the same rules (``load.py:77-132``): every layer listed in the
config must have its five required tensors (``KeyError`` when ``strict``, otherwise the layer
is skipped and reported as missing), ``padded_in_features`` is twice the packed width and the
group size comes from the layer entry, else the file-level entry, else 128.

Two deliberate differences: tensors are read one layer at a time through ``safe_open``
(the reference loads the whole file at once; the result is the same), and each layer's
tensor shapes are checked against its ``shape`` entry when it is read, so a malformed
checkpoint raises ``ValueError`` naming the layer at load time rather than at the first
forward.
"""
from __future__ import annotations

import json
from pathlib import Path

from safetensors import safe_open
from torch import nn

from ..config import BackendKind
from ..quant.state import SVDQuantLinearState
from .linear import SVDQuantLinear
from .replace import replace_module

CONFIG_NAME = "svdquant_config.json"
TENSORS_NAME = "transformer_svdquant.safetensors"
REQUIRED_SUFFIXES = ("qweight_packed", "weight_scales", "smooth_scale", "l1", "l2")


def _layer_key(layer_name: str) -> str:
    """Checkpoint key prefix of a dotted module name (reference ``load.py:16-17``)."""
    return layer_name.replace(".", "__")


def _resolve_checkpoint_dir(checkpoint_dir: str | Path) -> Path:
    """A local directory, or a Hugging Face repo id resolved through the local Hub snapshot.

    Same rule as reference ``load.py:20-49``: an existing path is used as is; a string that
    looks like ``owner/name`` (contains ``/`` and does not start with ``.``, ``/`` or ``~``)
    and is not a local path is fetched with ``huggingface_hub.snapshot_download``, limited to
    the two checkpoint files and the README.
    """
    path = Path(checkpoint_dir)
    if path.exists():
        return path
    repo_id = str(checkpoint_dir)
    if "/" not in repo_id or repo_id.startswith((".", "/", "~")):
        return path
    try:
        from huggingface_hub import snapshot_download
    except Exception as exc:  # environment without the Hub client
        raise FileNotFoundError(f"missing {path / CONFIG_NAME} and huggingface_hub is not installed; "
                                "pass a local checkpoint directory") from exc
    return Path(snapshot_download(repo_id=repo_id, repo_type="model",
                                  allow_patterns=[CONFIG_NAME, TENSORS_NAME, "README.md"]))


def _check_layer_shapes(layer_name: str, state: SVDQuantLinearState) -> None:
    n, k = state.original_shape
    g = state.group_size
    kp = state.padded_in_features
    problems = []
    if state.qweight.ndim != 2 or int(state.qweight.shape[0]) != n:
        problems.append(f"qweight_packed {tuple(state.qweight.shape)} is not [{n}, Kp/2]")
    if kp < k:
        problems.append(f"packed width covers {kp} inputs, fewer than K={k}")
    if g <= 0 or kp % g:
        problems.append(f"padded K={kp} is not a multiple of group_size={g}")
    elif tuple(state.weight_scales.shape) != (n, kp // g):
        problems.append(f"weight_scales {tuple(state.weight_scales.shape)} is not [{n}, {kp // g}]")
    if tuple(state.smooth_scale.shape) != (k,):
        problems.append(f"smooth_scale {tuple(state.smooth_scale.shape)} is not [{k}]")
    if state.l1.ndim != 2 or state.l2.ndim != 2 or int(state.l1.shape[0]) != n or \
            int(state.l2.shape[1]) != k or int(state.l1.shape[1]) != int(state.l2.shape[0]):
        problems.append(f"l1 {tuple(state.l1.shape)} / l2 {tuple(state.l2.shape)} are not [{n}, r] / [r, {k}]")
    if state.bias is not None and tuple(state.bias.shape) != (n,):
        problems.append(f"bias {tuple(state.bias.shape)} is not [{n}]")
    if problems:
        raise ValueError(f"checkpoint layer {layer_name}: " + "; ".join(problems))


def load_svdquant_transformer(transformer: nn.Module, checkpoint_dir: str | Path, *,
                              backend: BackendKind | str = BackendKind.AUTO, strict: bool = True) -> dict:
    """Replace every checkpoint layer of ``transformer`` with an ``SVDQuantLinear``.

    Returns the parsed ``svdquant_config.json`` with ``_load_report = {"replaced": [...],
    "missing": [...], "checkpoint_dir": str}`` added.  The tensors stay on the CPU, as in the
    reference; ``transformer.to(device)`` moves them, and each layer prepares its kernel
    operands on the device at its first forward.
    """
    root = _resolve_checkpoint_dir(checkpoint_dir)
    config_path, tensor_path = root / CONFIG_NAME, root / TENSORS_NAME
    for p in (config_path, tensor_path):
        if not p.exists():
            raise FileNotFoundError(f"missing {p}")
    config = json.loads(config_path.read_text())
    default_group = int(config.get("group_size", 128))
    replaced: list[str] = []
    missing: list[str] = []
    with safe_open(str(tensor_path), framework="pt", device="cpu") as f:
        present = set(f.keys())
        for layer_name, meta in config.get("layers", {}).items():
            key = _layer_key(layer_name)
            absent = [f"{key}.{s}" for s in REQUIRED_SUFFIXES if f"{key}.{s}" not in present]
            if absent:
                missing.extend(absent)
                if strict:
                    raise KeyError(f"missing tensors for {layer_name}: {absent}")
                continue
            n, k = (int(v) for v in meta["shape"])
            qweight = f.get_tensor(f"{key}.qweight_packed")
            state = SVDQuantLinearState(
                smooth_scale=f.get_tensor(f"{key}.smooth_scale"),
                qweight=qweight,
                weight_scales=f.get_tensor(f"{key}.weight_scales"),
                l1=f.get_tensor(f"{key}.l1"),
                l2=f.get_tensor(f"{key}.l2"),
                bias=f.get_tensor(f"{key}.bias") if f"{key}.bias" in present else None,
                group_size=int(meta.get("group_size", default_group)),
                original_shape=(n, k),
                qweight_packed=True,
                padded_in_features=int(qweight.shape[-1]) * 2,
            )
            _check_layer_shapes(layer_name, state)
            replace_module(transformer, layer_name, SVDQuantLinear(state, backend=backend))
            replaced.append(layer_name)
    if strict and missing:
        raise KeyError(f"missing tensors: {missing}")
    config["_load_report"] = {"replaced": replaced, "missing": missing, "checkpoint_dir": str(root)}
    return config


def save_transformer_checkpoint_readme(checkpoint_dir: str | Path, base_model: str) -> None:
    """Write the checkpoint's README (reference ``load.py:135-155``): what the directory holds
    and how to load it onto the base pipeline's transformer."""
    checkpoint_dir = Path(checkpoint_dir)
    text = (
        "# Krea2 SVDQuant transformer checkpoint\n\n"
        f"Transformer-only SVDQuant checkpoint for `{base_model}`: INT4 residual weights with "
        "fp16 group scales, bf16 smoothing scales and bf16 low-rank factors for each quantized "
        "linear. The text encoder, tokenizer, scheduler and VAE are not included; take them "
        "from the base model.\n\n"
        "```python\n"
        "import torch\n"
        "from diffusers import Krea2Pipeline\n"
        "from krea2_svdquant_amd.runtime.load import load_svdquant_transformer\n\n"
        f"pipe = Krea2Pipeline.from_pretrained(\"{base_model}\", torch_dtype=torch.bfloat16)\n"
        f"load_svdquant_transformer(pipe.transformer, \"{checkpoint_dir.name}\", backend=\"auto\")\n"
        "pipe.to(\"cuda\")\n"
        "```\n"
    )
    (checkpoint_dir / "README.md").write_text(text)
