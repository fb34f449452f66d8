"""Checkpoints in the reference's format, loaded without running code from the file.

Saving mirrors the reference's training loop (training/train.py:306-307,
:337-352): the model's state dict with every ``_orig_mod.`` prefix of a
``torch.compile``-wrapped model removed, written to ``path + ".tmp"`` and
moved into place, in a dict with ``model_state_dict``,
``optimizer_state_dict`` and the caller's extra entries (``step``,
``metrics``, ...).  A ``config`` dataclass is stored as a plain dict.

Loading reads the file with ``torch.load(weights_only=True)``: tensors,
containers and numbers only.  The reference also pickles its experiment
config (``training.training_config.LanguageModelingExperimentConfig`` holding
a ``src.config.ModelConfig`` and enums).  Those class names are mapped to
objects of this package before the load -- ``src.config.ModelConfig`` to
:class:`~outlierneuronattention_amd.config.ModelConfig`, every other class
the file names to :class:`OpaqueRecord`, which only stores the fields it is
given -- so the weights-only unpickler can rebuild them without importing or
calling anything from the reference.  Nothing is ever unpickled with
``weights_only=False``.

``load_model_state`` applies a state dict with the reference's
``strict=False`` semantics (src/inference.py:95-123): prefixes stripped,
missing and unexpected keys reported, and ``out_proj`` weights absent from
the checkpoint initialised to the identity.
"""
from __future__ import annotations

import dataclasses
import os
import pickle
import re
from typing import Any, Optional

import torch
import torch.nn as nn

from .config import ModelConfig

_PREFIX = "_orig_mod."


class OpaqueRecord:
    """Stand-in for a class a checkpoint names but this package does not
    define: keeps the constructor arguments (enums pickle as ``Cls(value)``)
    and the pickled instance state as plain data."""

    def __init__(self, *args):
        self.args = args

    def __setstate__(self, state):
        if isinstance(state, tuple) and len(state) == 2 and isinstance(state[0], (dict, type(None))):
            state = {**(state[0] or {}), **(state[1] or {})}
        if isinstance(state, dict):
            self.__dict__.update(state)
        else:
            self.state = state

    def __repr__(self):
        fields = {k: v for k, v in self.__dict__.items()}
        return f"OpaqueRecord({fields})"


def clean_state_dict(state: dict) -> dict:
    """Drop the ``_orig_mod.`` prefix a compiled model adds to every key
    (training/train.py:306-307)."""
    return {k.replace(_PREFIX, ""): v for k, v in state.items()}


def _plain(obj: Any) -> Any:
    if dataclasses.is_dataclass(obj) and not isinstance(obj, type):
        return {f.name: _plain(getattr(obj, f.name)) for f in dataclasses.fields(obj)}
    if isinstance(obj, dict):
        return {k: _plain(v) for k, v in obj.items()}
    if isinstance(obj, (list, tuple)):
        return type(obj)(_plain(v) for v in obj)
    return obj


def save_checkpoint(path: str, model: nn.Module, optimizer: Optional[torch.optim.Optimizer] = None,
                    config: Any = None, **extra) -> str:
    """Write ``{'model_state_dict', 'optimizer_state_dict', 'config', **extra}``
    atomically (temporary file, then ``os.replace``)."""
    ckpt = {"model_state_dict": clean_state_dict(model.state_dict())}
    if optimizer is not None:
        ckpt["optimizer_state_dict"] = optimizer.state_dict()
    if config is not None:
        ckpt["config"] = _plain(config)
    ckpt.update(extra)
    tmp = path + ".tmp"
    torch.save(ckpt, tmp)
    os.replace(tmp, path)
    return path


_GLOBAL_RE = re.compile(r"GLOBAL ([A-Za-z_][\w.]*)")


def load_checkpoint(path: str, map_location: Any = "cpu", max_classes: int = 64) -> dict:
    """Read a checkpoint with the weights-only unpickler.  Class names the file
    references are bound to :class:`ModelConfig` (``src.config.ModelConfig``)
    or :class:`OpaqueRecord` (anything else); no code from the file runs."""
    mapped: list = []
    for _ in range(max_classes):
        try:
            with torch.serialization.safe_globals(mapped):
                return torch.load(path, map_location=map_location, weights_only=True)
        except pickle.UnpicklingError as e:
            names = [n for n in _GLOBAL_RE.findall(str(e)) if n not in {m[1] for m in mapped}]
            # only class names (CamelCase) are stood in for; a function the
            # file asks for (a pickled call) leaves the error standing
            if not names or any(not n.rsplit(".", 1)[-1][:1].isupper() for n in names):
                raise
            for name in names:
                cls = ModelConfig if name.endswith(".config.ModelConfig") else OpaqueRecord
                mapped.append((cls, name))
    raise pickle.UnpicklingError(f"{path}: more than {max_classes} classes to map")


def load_model_state(model: nn.Module, ckpt_or_state: Any, verbose: bool = False):
    """Apply a checkpoint (path, checkpoint dict or bare state dict) to
    ``model`` as the reference's InferenceEngine does
    (src/inference.py:95-123): prefixes stripped, ``strict=False``, and every
    ``out_proj`` Linear whose weights the checkpoint lacks set to the
    identity.  Returns ``(missing_keys, unexpected_keys)``."""
    ck = load_checkpoint(ckpt_or_state) if isinstance(ckpt_or_state, (str, os.PathLike)) else ckpt_or_state
    state = ck["model_state_dict"] if isinstance(ck, dict) and "model_state_dict" in ck else ck
    state = clean_state_dict(state)
    # per-channel index buffers of older reference modules (src/inference.py:99-105);
    # these modules route channels by position and keep no such buffers
    state = {k: v for k, v in state.items() if "_cached_outlier_idx" not in k and "_cached_inlier_idx" not in k}
    missing, unexpected = model.load_state_dict(state, strict=False)
    if any("out_proj" in k for k in missing):
        with torch.no_grad():
            for name, module in model.named_modules():
                if "out_proj" in name and isinstance(module, nn.Linear) and f"{name}.weight" in missing:
                    nn.init.eye_(module.weight)
                    if module.bias is not None:
                        nn.init.zeros_(module.bias)
    if verbose and (missing or unexpected):
        print("Missing keys:", missing)
        print("Unexpected keys:", unexpected)
    return missing, unexpected
