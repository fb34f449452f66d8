"""Checkpoints in the reference's format (training/train.py:306-352,
src/inference.py:95-123), on the CPU.

The reference pickles its experiment config: a dataclass from
``training.training_config`` holding a ``src.config.ModelConfig`` and a
``str``-mixin Enum.  These tests build stand-in classes under those module
names, write a checkpoint with the full pickler exactly as the reference's
loop lays it out, remove the stand-ins again, and read the file back with the
weights-only loader, which never imports them.
"""
import dataclasses
import enum
import os
import sys
import types

import pytest
import torch

from outlierneuronattention_amd.checkpoint import (
    OpaqueRecord, clean_state_dict, load_checkpoint, load_model_state, save_checkpoint)
from outlierneuronattention_amd.config import ModelConfig
from outlierneuronattention_amd.HybridOutlierFactorizedAttention import SubwordLM as InferLM
from outlierneuronattention_amd.HybridOutlierFactorizedAttentionTrain import SubwordLM as TrainLM

CFG = dict(d_model=64, num_heads=2, num_layers=2, r=[8, 16], block_size=64, device="cpu")


def _reference_like_modules():
    """Stand-ins for ``src.config`` and ``training.training_config`` with the
    reference's class names and field layout."""
    src = types.ModuleType("src")
    src_config = types.ModuleType("src.config")
    training = types.ModuleType("training")
    tcfg = types.ModuleType("training.training_config")

    @dataclasses.dataclass
    class ModelConfigRef:
        d_model: int = 384
        num_heads: int = 6
        num_layers: int = 6
        r: object = 8
        block_size: int = 1024
        learnable_alpha: bool = False

    ModelConfigRef.__name__ = ModelConfigRef.__qualname__ = "ModelConfig"
    ModelConfigRef.__module__ = "src.config"
    src_config.ModelConfig = ModelConfigRef

    class DatasetType(str, enum.Enum):
        FINEWEB = "fineweb"
        PG19 = "pg19"

    DatasetType.__module__ = "training.training_config"
    DatasetType.__qualname__ = "DatasetType"

    @dataclasses.dataclass
    class LanguageModelingExperimentConfig:
        model_name: str = "30M_HOFA"
        model_config: ModelConfigRef = None
        dataset_name: DatasetType = DatasetType.FINEWEB
        seq_len: int = 1024

    LanguageModelingExperimentConfig.__module__ = "training.training_config"
    LanguageModelingExperimentConfig.__qualname__ = "LanguageModelingExperimentConfig"
    tcfg.DatasetType = DatasetType
    tcfg.LanguageModelingExperimentConfig = LanguageModelingExperimentConfig
    return {"src": src, "src.config": src_config, "training": training,
            "training.training_config": tcfg}


def _write_reference_checkpoint(path, model, optimizer):
    mods = _reference_like_modules()
    saved = {k: sys.modules.get(k) for k in mods}
    sys.modules.update(mods)
    try:
        tc = mods["training.training_config"]
        mc = mods["src.config"].ModelConfig(d_model=64, num_heads=2, num_layers=2, r=[8, 16], block_size=64)
        config = tc.LanguageModelingExperimentConfig(model_name="30M_HOFA", model_config=mc)
        # a compiled model's keys carry ``_orig_mod.``; the reference strips them before saving
        raw = {"_orig_mod." + k: v for k, v in model.state_dict().items()}
        torch.save({
            "model_state_dict": {k.replace("_orig_mod.", ""): v for k, v in raw.items()},
            "optimizer_state_dict": optimizer.state_dict(),
            "config": config,
            "metrics": {"train_loss": [3.5, 3.25], "val_ppl": [40.0]},
            "step": 250,
            "start_idx": 12345,
            "total_processed_tokens": 1 << 20,
            "best_val_ppl": 40.0,
            "rng_state": torch.get_rng_state(),
            "cuda_rng_state": [],
        }, path)
    finally:
        for k, v in saved.items():
            if v is None:
                sys.modules.pop(k, None)
            else:
                sys.modules[k] = v


@pytest.fixture
def train_model():
    torch.manual_seed(0)
    return TrainLM(100, ModelConfig(**CFG))


def test_reference_checkpoint_loads_weights_only(tmp_path, train_model):
    opt = torch.optim.AdamW(train_model.parameters(), lr=1e-3)
    path = str(tmp_path / "checkpoint.pt")
    _write_reference_checkpoint(path, train_model, opt)
    assert "src.config" not in sys.modules and "training.training_config" not in sys.modules

    ck = load_checkpoint(path)
    assert ck["step"] == 250 and ck["start_idx"] == 12345
    assert ck["metrics"]["val_ppl"] == [40.0]
    cfg = ck["config"]
    assert isinstance(cfg, OpaqueRecord)
    assert cfg.model_name == "30M_HOFA"
    assert isinstance(cfg.model_config, ModelConfig)
    assert cfg.model_config.r == [8, 16] and cfg.model_config.d_model == 64
    assert isinstance(cfg.dataset_name, OpaqueRecord) and cfg.dataset_name.args == ("fineweb",)
    # nothing from the stand-in modules was imported by the load
    assert "src.config" not in sys.modules and "training.training_config" not in sys.modules

    for cls in (TrainLM, InferLM):
        torch.manual_seed(1)
        m = cls(100, ModelConfig(**CFG))
        missing, unexpected = load_model_state(m, path)
        assert missing == [] and unexpected == []
        for k, v in train_model.state_dict().items():
            assert torch.equal(m.state_dict()[k], v), k


def test_full_pickle_is_never_used(tmp_path, train_model, monkeypatch):
    """The loader goes through ``weights_only=True`` on every attempt."""
    path = str(tmp_path / "ck.pt")
    _write_reference_checkpoint(path, train_model, torch.optim.SGD(train_model.parameters(), lr=0.1))
    calls = []
    real = torch.load

    def spy(*a, **kw):
        calls.append(kw.get("weights_only"))
        return real(*a, **kw)

    monkeypatch.setattr(torch, "load", spy)
    load_checkpoint(path)
    assert calls and all(w is True for w in calls)


def test_code_in_a_checkpoint_is_not_run(tmp_path):
    """A file that asks the unpickler to call a function is refused, not run."""

    class Boom:
        def __reduce__(self):
            return (os.system, ("echo pwned > " + str(tmp_path / "ran"),))

    path = str(tmp_path / "evil.pt")
    torch.save({"model_state_dict": {}, "x": Boom()}, path)
    with pytest.raises(Exception):
        load_checkpoint(path)
    assert not (tmp_path / "ran").exists()


def test_orig_mod_prefix_and_identity_out_proj(train_model):
    state = {"_orig_mod." + k: v for k, v in train_model.state_dict().items()}
    assert all(not k.startswith("_orig_mod.") for k in clean_state_dict(state))
    dropped = [k for k in state if "layers.1.attn.out_proj" in k]
    assert dropped
    for k in dropped:
        del state[k]
    torch.manual_seed(2)
    m = TrainLM(100, ModelConfig(**CFG))
    missing, unexpected = load_model_state(m, {"model_state_dict": state})
    assert sorted(missing) == sorted(k.replace("_orig_mod.", "") for k in dropped)
    assert unexpected == []
    w = m.layers[1].attn.out_proj.weight
    assert torch.equal(w, torch.eye(*w.shape))
    # the layer whose out_proj the checkpoint holds keeps its weights
    assert torch.equal(m.layers[0].attn.out_proj.weight, train_model.layers[0].attn.out_proj.weight)


def test_cached_index_buffers_are_ignored(train_model):
    state = dict(train_model.state_dict())
    state["layers.0.attn._cached_outlier_idx"] = torch.arange(8)
    state["layers.0.attn._cached_inlier_idx"] = torch.arange(8, 32)
    m = TrainLM(100, ModelConfig(**CFG))
    missing, unexpected = load_model_state(m, state)
    assert missing == [] and unexpected == []


def test_save_roundtrip(tmp_path, train_model):
    path = str(tmp_path / "ours.pt")
    save_checkpoint(path, train_model, torch.optim.AdamW(train_model.parameters()),
                    config=ModelConfig(**CFG), step=7)
    assert not os.path.exists(path + ".tmp")
    ck = load_checkpoint(path)
    assert ck["step"] == 7 and ck["config"]["r"] == [8, 16]
    m = InferLM(100, ModelConfig(**CFG))
    assert load_model_state(m, path) == ([], [])
    for k, v in train_model.state_dict().items():
        assert torch.equal(m.state_dict()[k], v)


def test_pickled_function_call_is_refused(tmp_path):
    """A call to an importable function (not a class) is refused too."""

    class Call:
        def __reduce__(self):
            return (print, ("ran",))

    path = str(tmp_path / "call.pt")
    torch.save({"x": Call()}, path)
    with pytest.raises(Exception):
        load_checkpoint(path)
