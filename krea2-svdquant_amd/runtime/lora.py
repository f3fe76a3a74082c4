"""Attaching the adapters of a LoRA file to the ``SVDQuantLinear`` modules of a transformer.

Public behaviour follows reference ``src/krea2_svdquant/runtime/lora.py:135-187``
(``load_svdquant_lora_adapters``): every complete down/up pair of the file is attached to the one
quantized module its name designates, with ``add_lora_adapter`` (here the adapter then runs fused
inside the two kernels: down projection in the activation pass, up projection in the GEMM
epilogue), and a report ``{"lora_file", "loaded", "unmatched", "incomplete"}`` is returned.

How it works:

* ``resolve_lora_file`` turns the argument into one file: the file itself; in a directory the
  ``weight_name`` given, else the first of ``COMMON_WEIGHT_NAMES`` present, else the only
  ``*.safetensors``; otherwise the argument is taken as a Hub repo id (reference ``:37-73``).
* ``parse_key`` splits a tensor key into adapter name and role with one regular expression over
  the suffix tables; the name is the shortest prefix, so the longest (most specific) suffix wins
  (``a.lora.down.weight`` names adapter ``a``, not ``a.lora``).  An alpha tensor of more than one
  element counts as absent, and ``network_alpha`` then defaults to the rank (reference ``:116-132``).
* ``ModuleIndex`` indexes the model's quantized modules by dotted name and by the name with every
  ``.`` turned into ``_``.  An adapter name, after the leading ``KNOWN_PREFIXES`` are stripped,
  designates a module when one of its dotted suffixes (split at ``.``) is the module's name, or one
  of its underscore suffixes is the module's flat name (Kohya keys such as
  ``lora_unet_transformer_blocks_0_attn_to_q``; reference ``:87-113``).  Every candidate is one
  dictionary lookup.
* A name that designates two modules raises ``ValueError``; with ``strict``, a file that attaches
  nothing raises ``ValueError``.

``.bin`` / ``.pt`` files are read with ``torch.load(weights_only=True)`` (tensors and plain
containers only), unwrapping a ``{"state_dict": ...}`` container.
"""
from __future__ import annotations

import re
from collections import defaultdict
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Iterator, Mapping, Optional

import torch
from safetensors.torch import load_file

from .linear import SVDQuantLinear

# Format tables: the spellings LoRA files use for their weight files, tensor-key suffixes and
# framework prefixes.
COMMON_WEIGHT_NAMES = (
    "pytorch_lora_weights.safetensors",
    "adapter_model.safetensors",
    "lora.safetensors",
    "pytorch_lora_weights.bin",
    "adapter_model.bin",
)
DOWN_SUFFIXES = (".lora_A.weight", ".lora.down.weight", ".lora_linear_layer.down.weight",
                 ".lora_down.weight", ".down.weight")
UP_SUFFIXES = (".lora_B.weight", ".lora.up.weight", ".lora_linear_layer.up.weight",
               ".lora_up.weight", ".up.weight")
ALPHA_SUFFIXES = (".alpha", ".network_alpha", ".lora_alpha")
KNOWN_PREFIXES = ("transformer.", "unet.", "base_model.model.", "model.", "module.", "diffusion_model.")

_ROLES = {**{s: "down" for s in DOWN_SUFFIXES}, **{s: "up" for s in UP_SUFFIXES},
          **{s: "alpha" for s in ALPHA_SUFFIXES}}
_KEY = re.compile(r"(?P<name>.+?)(?P<suffix>%s)" % "|".join(re.escape(s) for s in _ROLES))
_PREFIXES = re.compile(r"(?:%s)+" % "|".join(re.escape(p) for p in KNOWN_PREFIXES))


# ----------------------------------------------------------------------------- file
def _file_in_directory(directory: Path, weight_name: Optional[str]) -> Path:
    if weight_name is not None:
        chosen = directory / weight_name
        if not chosen.exists():
            raise FileNotFoundError(chosen)
        return chosen
    usual = [directory / n for n in COMMON_WEIGHT_NAMES if (directory / n).exists()]
    if usual:
        return usual[0]
    tensors = sorted(directory.glob("*.safetensors"))
    if len(tensors) != 1:
        raise FileNotFoundError(f"could not infer the LoRA file in {directory} ({len(tensors)} *.safetensors "
                                "files, none of the usual names); pass weight_name")
    return tensors[0]


def _file_on_hub(repo_id: str, weight_name: Optional[str]) -> Path:
    try:
        from huggingface_hub import hf_hub_download
    except Exception as exc:  # environment without the Hub client
        raise ImportError(f"loading LoRA {repo_id!r} from the Hub needs huggingface_hub") from exc
    error: Optional[Exception] = None
    for name in (weight_name,) if weight_name is not None else COMMON_WEIGHT_NAMES:
        try:
            return Path(hf_hub_download(repo_id=repo_id, filename=name, repo_type="model"))
        except Exception as exc:  # the next usual name may exist
            error = exc
    raise FileNotFoundError(f"no LoRA weight file found in Hub repo {repo_id}") from error


def resolve_lora_file(source: str | Path, weight_name: Optional[str] = None) -> Path:
    """The one LoRA weight file that ``source`` (file, directory or Hub repo id) designates."""
    path = Path(source).expanduser()
    if path.is_file():
        return path
    if path.is_dir():
        return _file_in_directory(path, weight_name)
    repo_id = str(source)
    looks_local = repo_id.startswith((".", "/", "~")) or "/" not in repo_id
    if looks_local:
        raise FileNotFoundError(path)
    return _file_on_hub(repo_id, weight_name)


def read_lora_tensors(path: Path) -> dict[str, torch.Tensor]:
    """The tensors of a LoRA file (safetensors, or a torch pickle read with weights_only=True)."""
    if path.suffix == ".safetensors":
        return load_file(str(path), device="cpu")
    obj = torch.load(path, map_location="cpu", weights_only=True)
    if isinstance(obj, dict) and isinstance(obj.get("state_dict"), dict):
        obj = obj["state_dict"]
    if not isinstance(obj, dict):
        raise TypeError(f"{path} holds a {type(obj).__name__}, not a dict of LoRA tensors")
    return {str(k): v for k, v in obj.items() if torch.is_tensor(v)}


# ----------------------------------------------------------------------------- keys
def parse_key(key: str) -> Optional[tuple[str, str]]:
    """``(adapter name, "down" | "up" | "alpha")`` of a LoRA tensor key, or None."""
    m = _KEY.fullmatch(key)
    return (m.group("name"), _ROLES[m.group("suffix")]) if m else None


def canonical_name(name: str) -> str:
    """``name`` without its leading framework prefixes (all of them, in any order)."""
    m = _PREFIXES.match(name)
    return name[m.end():] if m else name


@dataclass
class AdapterEntry:
    """One adapter of a LoRA file: its name and the parts the file holds."""
    name: str
    down: Optional[torch.Tensor] = None
    up: Optional[torch.Tensor] = None
    alpha: Optional[float] = None

    @property
    def complete(self) -> bool:
        return self.down is not None and self.up is not None


def group_adapters(tensors: Mapping[str, torch.Tensor]) -> dict[str, AdapterEntry]:
    """The adapters of a LoRA state dict by name, in the order their names first appear."""
    entries: dict[str, AdapterEntry] = {}
    for key, tensor in tensors.items():
        parsed = parse_key(key)
        if parsed is None:
            continue
        name, role = parsed
        entry = entries.setdefault(name, AdapterEntry(name))
        if role == "alpha":
            entry.alpha = float(tensor.item()) if tensor.numel() == 1 else None
        else:
            setattr(entry, role, tensor)
    return entries


def _suffixes(name: str, sep: str) -> Iterator[str]:
    """``name`` and every tail of it that starts right after a ``sep``."""
    yield name
    pos = name.find(sep)
    while pos >= 0:
        yield name[pos + 1:]
        pos = name.find(sep, pos + 1)


class ModuleIndex:
    """The ``SVDQuantLinear`` modules of a model, looked up by the names LoRA files give them."""

    def __init__(self, root: torch.nn.Module):
        self.modules = {n: m for n, m in root.named_modules() if isinstance(m, SVDQuantLinear)}
        self._order = {n: i for i, n in enumerate(self.modules)}
        self._dotted = {n: n for n in self.modules}
        self._flat: dict[str, list[str]] = defaultdict(list)
        for n in self.modules:
            self._flat[n.replace(".", "_")].append(n)

    def matches(self, adapter_name: str) -> list[str]:
        """Module names the adapter name designates (module order)."""
        key = canonical_name(adapter_name)
        hits = {self._dotted[s] for s in _suffixes(key, ".") if s in self._dotted}
        for s in _suffixes(key.replace(".", "_"), "_"):
            hits.update(self._flat.get(s, ()))
        return sorted(hits, key=self._order.__getitem__)


# ----------------------------------------------------------------------------- loader
def load_svdquant_lora_adapters(transformer: torch.nn.Module, lora_path_or_repo_id: str | Path, *,
                                weight_name: Optional[str] = None, scale: float = 1.0,
                                strict: bool = True) -> dict[str, Any]:
    """Attach every adapter of a LoRA file to the ``SVDQuantLinear`` of ``transformer`` it names.

    ``scale`` multiplies every adapter (``multiplier = scale * alpha / rank``).  Returns
    ``{"lora_file", "loaded", "unmatched", "incomplete"}``: the modules that received an adapter,
    and the adapter names that designate no module or lack their down or up weight.
    """
    path = resolve_lora_file(lora_path_or_repo_id, weight_name=weight_name)
    index = ModuleIndex(transformer)
    report: dict[str, Any] = {"lora_file": str(path), "loaded": [], "unmatched": [], "incomplete": []}
    for entry in group_adapters(read_lora_tensors(path)).values():
        if not entry.complete:
            report["incomplete"].append(entry.name)
            continue
        targets = index.matches(entry.name)
        if len(targets) > 1:
            raise ValueError(f"LoRA adapter {entry.name!r} matches multiple modules: {targets}")
        if not targets:
            report["unmatched"].append(entry.name)
            continue
        index.modules[targets[0]].add_lora_adapter(entry.down, entry.up, scale=scale, network_alpha=entry.alpha)
        report["loaded"].append(targets[0])
    if strict and not report["loaded"]:
        raise ValueError(f"no LoRA tensors in {path} attach to an SVDQuantLinear of this model "
                         f"({len(report['unmatched'])} unmatched, {len(report['incomplete'])} incomplete adapters); "
                         "is it a LoRA for this transformer, and is weight_name right?")
    return report
