"""Processor installation on a model (dfsattn/attn_processor.py:5-61).

``get_attn_processors`` / ``set_attn_processor`` walk the module tree and
talk to every module that has ``get_processor`` / ``set_processor`` (the
diffusers ``Attention`` protocol), keyed by ``"<module path>.processor"``.
"""
from __future__ import annotations

from typing import Any, Dict, Union

import torch


def get_attn_processors(module: torch.nn.Module) -> Dict[str, Any]:
    """{"<path>.processor": processor} for every attention module."""
    found: Dict[str, Any] = {}

    def visit(name: str, mod: torch.nn.Module) -> None:
        if hasattr(mod, "get_processor"):
            found[f"{name}.processor"] = mod.get_processor()
        for child_name, child in mod.named_children():
            visit(f"{name}.{child_name}", child)

    for name, child in module.named_children():
        visit(name, child)
    return found


def set_attn_processor(module: torch.nn.Module, processor: Union[Any, Dict[str, Any]]) -> None:
    """Installs one processor on every attention module, or a dict of them
    keyed as ``get_attn_processors`` returns (consumed as it is applied)."""
    count = len(get_attn_processors(module))
    if isinstance(processor, dict) and len(processor) != count:
        raise ValueError(
            f"A dict of processors was passed, but the number of processors {len(processor)} does not match the"
            f" number of attention layers: {count}. Please make sure to pass {count} processor classes.")

    def visit(name: str, mod: torch.nn.Module) -> None:
        if hasattr(mod, "set_processor"):
            mod.set_processor(processor.pop(f"{name}.processor") if isinstance(processor, dict) else processor)
        for child_name, child in mod.named_children():
            visit(f"{name}.{child_name}", child)

    for name, child in module.named_children():
        visit(name, child)
