"""Locating and swapping linears inside a module tree by dotted name.

Same three helpers and behaviour as reference ``src/krea2_svdquant/runtime/replace.py:10-30``:
``iter_named_linears`` yields the ``nn.Linear`` modules whose dotted name ends with one of the
target suffixes (default: ``SVDQuantConfig().target_modules``), ``get_parent_module`` walks a
dotted name (numeric parts index ``ModuleList``/``Sequential`` children) and
``replace_module`` installs a new module at that name.
"""
from __future__ import annotations

from collections.abc import Iterable, Iterator

from torch import nn

from ..config import SVDQuantConfig


def iter_named_linears(root: nn.Module, target_suffixes: Iterable[str] | None = None
                       ) -> Iterator[tuple[str, nn.Linear]]:
    suffixes = tuple(target_suffixes) if target_suffixes else SVDQuantConfig().target_modules
    for name, module in root.named_modules():
        if isinstance(module, nn.Linear) and name.endswith(suffixes):
            yield name, module


def get_parent_module(root: nn.Module, dotted_name: str) -> tuple[nn.Module, str]:
    *path, leaf = dotted_name.split(".")
    node = root
    for part in path:
        node = node[int(part)] if part.isdigit() else getattr(node, part)
    return node, leaf


def replace_module(root: nn.Module, dotted_name: str, new_module: nn.Module) -> None:
    parent, leaf = get_parent_module(root, dotted_name)
    if leaf.isdigit():
        parent[int(leaf)] = new_module
    else:
        setattr(parent, leaf, new_module)
