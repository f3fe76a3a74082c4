"""LoRA files onto a quantized transformer: each adapter pair attaches to its ``SVDQuantLinear``.

Mirror of reference ``src/krea2_svdquant/runtime/lora.py``.  Diffusers/PEFT would inject
adapters into ``nn.Linear`` modules that the SVDQuant checkpoint has already replaced, so the
pairs are matched to ``SVDQuantLinear`` modules by name and attached with
``add_lora_adapter``; in this package the adapter then runs fused inside the two kernels
(down projection in the activation pass, up projection in the GEMM epilogue).

Behaviour kept from the reference:

* file resolution (``lora.py:37-73``): a file path; a directory with ``weight_name`` or one of
  the usual file names or exactly one ``*.safetensors``; else a Hub repo id;
* key grammar (``lora.py:20-34,116-132``): a tensor is a down weight, an up weight or an alpha
  by its suffix, and the rest of the key names the adapter; an alpha of more than one element
  counts as absent (``network_alpha`` then defaults to the rank);
* name matching (``lora.py:87-113``): leading ``transformer.``, ``unet.``,
  ``base_model.model.``, ``model.``, ``module.``, ``diffusion_model.`` are stripped
  repeatedly; the rest must equal the module name or end with ``.<module name>``, or, with
  every ``.`` turned into ``_``, equal it or end with ``_<module name>`` (Kohya names such as
  ``lora_unet_transformer_blocks_0_attn_to_q``);
* outcome (``lora.py:152-187``): pairs missing a half are reported as incomplete, names that
  match nothing as unmatched, a name that matches several modules raises ``ValueError``, and
  with ``strict`` a file that attaches nothing raises ``ValueError``.

One deliberate difference: ``.bin`` / ``.pt`` files are read with
``torch.load(weights_only=True)``, which accepts tensors and plain containers only.
"""
from __future__ import annotations

from collections import defaultdict
from pathlib import Path
from typing import Any

import torch
from safetensors.torch import load_file

from .linear import SVDQuantLinear

COMMON_WEIGHT_NAMES = (
    "pytorch_lora_weights.safetensors",
    "adapter_model.safetensors",
    "lora.safetensors",
    "pytorch_lora_weights.bin",
    "adapter_model.bin",
)
# Suffix lists are tried in order; the more specific spellings come before ".down.weight" /
# ".up.weight", which they also end with.
DOWN_SUFFIXES = (".lora_A.weight", ".lora.down.weight", ".lora_linear_layer.down.weight",
                 ".lora_down.weight", ".down.weight")
UP_SUFFIXES = (".lora_B.weight", ".lora.up.weight", ".lora_linear_layer.up.weight",
               ".lora_up.weight", ".up.weight")
ALPHA_SUFFIXES = (".alpha", ".network_alpha", ".lora_alpha")
KNOWN_PREFIXES = ("transformer.", "unet.", "base_model.model.", "model.", "module.", "diffusion_model.")


def _resolve_lora_file(lora_path_or_repo_id: str | Path, weight_name: str | None = None) -> Path:
    path = Path(lora_path_or_repo_id).expanduser()
    if path.is_file():
        return path
    if path.is_dir():
        if weight_name is not None:
            chosen = path / weight_name
            if not chosen.exists():
                raise FileNotFoundError(chosen)
            return chosen
        for name in COMMON_WEIGHT_NAMES:
            if (path / name).exists():
                return path / name
        found = sorted(path.glob("*.safetensors"))
        if len(found) == 1:
            return found[0]
        raise FileNotFoundError(f"could not infer LoRA weight file in {path}; pass weight_name")
    repo_id = str(lora_path_or_repo_id)
    if "/" not in repo_id or repo_id.startswith((".", "/", "~")):
        raise FileNotFoundError(path)
    try:
        from huggingface_hub import hf_hub_download
    except Exception as exc:  # environment without the Hub client
        raise ImportError("huggingface_hub is required to load LoRA weights from the Hub") from exc
    last_error: Exception | None = None
    for name in ((weight_name,) if weight_name is not None else COMMON_WEIGHT_NAMES):
        try:
            return Path(hf_hub_download(repo_id=repo_id, filename=name, repo_type="model"))
        except Exception as exc:  # try the next usual name
            last_error = exc
    raise FileNotFoundError(f"could not find a LoRA weight file in Hub repo {repo_id}") from last_error


def _load_lora_state_dict(path: Path) -> dict[str, torch.Tensor]:
    if path.suffix == ".safetensors":
        return load_file(str(path), device="cpu")
    state = torch.load(path, map_location="cpu", weights_only=True)
    if isinstance(state, dict) and isinstance(state.get("state_dict"), dict):
        state = state["state_dict"]
    if not isinstance(state, dict):
        raise TypeError(f"unsupported LoRA checkpoint format: {path}")
    return {str(k): v for k, v in state.items() if torch.is_tensor(v)}


def _strip_known_prefixes(name: str) -> str:
    stripped = True
    while stripped:
        stripped = False
        for prefix in KNOWN_PREFIXES:
            if name.startswith(prefix):
                name = name[len(prefix):]
                stripped = True
    return name


def _module_matches(prefix: str, module_name: str) -> bool:
    prefix = _strip_known_prefixes(prefix)
    if prefix == module_name or prefix.endswith("." + module_name):
        return True
    flat_prefix, flat_module = prefix.replace(".", "_"), module_name.replace(".", "_")
    return flat_prefix == flat_module or flat_prefix.endswith("_" + flat_module)


def _match_suffix(key: str, suffixes: tuple[str, ...]) -> str | None:
    for suffix in suffixes:
        if key.endswith(suffix):
            return key[: -len(suffix)]
    return None


def _split_lora_pairs(state_dict: dict[str, torch.Tensor]) -> dict[str, dict[str, Any]]:
    """Group a LoRA state dict by adapter name: ``{name: {"down", "up", "alpha"}}`` (each part
    present when the file has it), in the order the names first appear."""
    pairs: dict[str, dict[str, Any]] = defaultdict(dict)
    for key, tensor in state_dict.items():
        name = _match_suffix(key, DOWN_SUFFIXES)
        if name is not None:
            pairs[name]["down"] = tensor
        name = _match_suffix(key, UP_SUFFIXES)
        if name is not None:
            pairs[name]["up"] = tensor
        name = _match_suffix(key, ALPHA_SUFFIXES)
        if name is not None:
            pairs[name]["alpha"] = tensor.item() if tensor.numel() == 1 else None
    return pairs


def load_svdquant_lora_adapters(transformer: torch.nn.Module, lora_path_or_repo_id: str | Path, *,
                                weight_name: str | None = None, scale: float = 1.0,
                                strict: bool = True) -> dict[str, Any]:
    """Attach every adapter pair of a LoRA file to the matching ``SVDQuantLinear`` of ``transformer``.

    Returns ``{"lora_file", "loaded", "unmatched", "incomplete"}`` like the reference.
    ``scale`` multiplies every adapter (``multiplier = scale * alpha / rank``).
    """
    lora_file = _resolve_lora_file(lora_path_or_repo_id, weight_name=weight_name)
    pairs = _split_lora_pairs(_load_lora_state_dict(lora_file))
    modules = {name: mod for name, mod in transformer.named_modules() if isinstance(mod, SVDQuantLinear)}
    loaded: list[str] = []
    unmatched: list[str] = []
    incomplete: list[str] = []
    for prefix, parts in pairs.items():
        if "down" not in parts or "up" not in parts:
            incomplete.append(prefix)
            continue
        hits = [name for name in modules if _module_matches(prefix, name)]
        if not hits:
            unmatched.append(prefix)
            continue
        if len(hits) > 1:
            raise ValueError(f"LoRA prefix {prefix!r} matched multiple modules: {hits}")
        modules[hits[0]].add_lora_adapter(parts["down"], parts["up"], scale=scale,
                                          network_alpha=parts.get("alpha"))
        loaded.append(hits[0])
    if strict and not loaded:
        raise ValueError(f"no LoRA tensors from {lora_file} matched SVDQuant transformer layers; "
                         "check that this is a Krea2 transformer LoRA or pass the right weight_name")
    return {"lora_file": str(lora_file), "loaded": loaded, "unmatched": unmatched, "incomplete": incomplete}
