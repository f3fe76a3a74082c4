"""Finding the target linears of a transformer and installing modules in their place.

The public names are those of reference ``src/krea2_svdquant/runtime/replace.py:10-30`` (callers
import them): ``iter_named_linears`` lists the ``nn.Linear`` modules whose dotted name ends with a
target suffix (default: ``SVDQuantConfig().target_modules``), ``get_parent_module`` splits a dotted
name into its owner module and attribute, ``replace_module`` installs a new module there.

Both lookups go through ``nn.Module.get_submodule``: the children of ``nn.ModuleList`` /
``nn.Sequential`` are registered under their decimal index, so a dotted path such as
``transformer_blocks.3.attn.to_out.0`` resolves without special cases, and assigning to such an
index name with ``setattr`` replaces the list entry.
"""
from __future__ import annotations

from collections.abc import Iterable, Iterator

from torch import nn

from ..config import SVDQuantConfig


def iter_named_linears(root: nn.Module, target_suffixes: Iterable[str] | None = None
                       ) -> Iterator[tuple[str, nn.Linear]]:
    """``(dotted name, module)`` of every ``nn.Linear`` under ``root`` whose name ends with one
    of ``target_suffixes``, in ``named_modules`` order."""
    wanted = tuple(target_suffixes or SVDQuantConfig().target_modules)
    return ((name, mod) for name, mod in root.named_modules()
            if isinstance(mod, nn.Linear) and name.endswith(wanted))


def get_parent_module(root: nn.Module, dotted_name: str) -> tuple[nn.Module, str]:
    """The module that owns ``dotted_name`` and the attribute (or index) name under it."""
    owner, _, attr = dotted_name.rpartition(".")
    return root.get_submodule(owner), attr


def replace_module(root: nn.Module, dotted_name: str, new_module: nn.Module) -> None:
    """Install ``new_module`` at ``dotted_name`` (list / sequential entries included)."""
    parent, attr = get_parent_module(root, dotted_name)
    if not hasattr(parent, attr):
        raise AttributeError(f"{type(parent).__name__} has no child {attr!r} ({dotted_name})")
    setattr(parent, attr, new_module)
