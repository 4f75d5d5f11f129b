"""State-dict / export compatibility and metric-history format (CPU).

The reference validates an exported GPT state against the keys and shapes of
a freshly built model (inference/artifact.py:392-420, 423-435) and writes it
with ``torch.save`` (artifact.py:599); its metric history is versioned JSONL
(training/metric_history.py).  These tests hold this package's model and
metrics to the same contracts.
"""

from __future__ import annotations

import io
import json
import math

import pytest
import torch

import nano_megatron_amd as nm
from nano_megatron_amd import metrics as M
from oracle import reference as R


def reference_state_shapes(cfg: nm.GPTConfig) -> dict[str, tuple[int, ...]]:
    """Keys and shapes of the reference GPTModel's state_dict at TP=1, read off
    its modules: embedding / final_norm / tied lm_head (models/gpt/model.py:86-142),
    per layer input_norm, attention, post_attention_norm, mlp (layer.py:47-61), the
    projections as ``<name>.linear.weight`` (attention.py:82-117, mlp.py:44-70,
    tensor_parallel/layers.py:56-70, 112-132) with, under ``bias``, the column
    projections' ``<name>.linear.bias`` and the row projections' ``<name>.bias``
    (layers.py:110-126), no persistent buffers (the RoPE inv_freq is
    non-persistent, nn/rotary.py:53); ``lm_head.weight`` is the embedding's
    when tied, its own tensor otherwise (model.py:125-142)."""
    h, v, f = cfg.hidden_size, cfg.vocab_size, cfg.ffn_hidden_size
    hq = cfg.heads
    hkv = cfg.kv_heads or hq
    d = h // hq
    shapes: dict[str, tuple[int, ...]] = {"embedding.weight": (v, h)}
    for i in range(cfg.layers):
        p = f"layers.{i}."
        shapes[p + "input_norm.weight"] = (h,)
        shapes[p + "attention.q_proj.linear.weight"] = (hq * d, h)
        shapes[p + "attention.k_proj.linear.weight"] = (hkv * d, h)
        shapes[p + "attention.v_proj.linear.weight"] = (hkv * d, h)
        shapes[p + "attention.out_proj.linear.weight"] = (h, hq * d)
        shapes[p + "post_attention_norm.weight"] = (h,)
        shapes[p + "mlp.gate_proj.linear.weight"] = (f, h)
        shapes[p + "mlp.up_proj.linear.weight"] = (f, h)
        shapes[p + "mlp.down_proj.linear.weight"] = (h, f)
        if cfg.bias:
            for name, n in (("attention.q_proj", hq * d), ("attention.k_proj", hkv * d),
                            ("attention.v_proj", hkv * d), ("mlp.gate_proj", f), ("mlp.up_proj", f)):
                shapes[p + name + ".linear.bias"] = (n,)
            shapes[p + "attention.out_proj.bias"] = (h,)
            shapes[p + "mlp.down_proj.bias"] = (h,)
    shapes["final_norm.weight"] = (h,)
    shapes["lm_head.weight"] = (v, h)
    return shapes


CONFIGS = [
    dict(layers=2, hidden_size=128, ffn_hidden_size=352, heads=2, seq_length=32, vocab_size=256),
    dict(layers=3, hidden_size=256, ffn_hidden_size=688, heads=4, kv_heads=2, seq_length=32, vocab_size=512),
    dict(layers=2, hidden_size=128, ffn_hidden_size=352, heads=2, seq_length=32, vocab_size=256, bias=True,
         tie_embeddings=False),
]


def _validate_like_export(state: dict, cfg: nm.GPTConfig) -> None:
    """The checks of artifact.py:392-420 on a merged state."""
    expected = reference_state_shapes(cfg)
    assert set(state) == set(expected), (set(state) ^ set(expected))
    for key, shape in expected.items():
        assert tuple(state[key].shape) == shape, key
    floating = {t.dtype for t in state.values() if t.is_floating_point()}
    assert len(floating) == 1
    assert state["embedding.weight"].dtype == state["lm_head.weight"].dtype
    if cfg.tie_embeddings:
        assert torch.equal(state["embedding.weight"], state["lm_head.weight"])


@pytest.mark.parametrize("kw", CONFIGS)
def test_state_dict_keys_and_shapes_match_the_reference(kw) -> None:
    cfg = nm.GPTConfig(**kw)
    state = nm.GPTModel(cfg).state_dict()
    assert {k: tuple(t.shape) for k, t in state.items()} == reference_state_shapes(cfg)
    # the CPU oracle (a restatement of the reference modules) has the same state layout
    oracle = R.OracleGPTModel(cfg).state_dict()
    assert {k: tuple(t.shape) for k, t in oracle.items()} == reference_state_shapes(cfg)


@pytest.mark.parametrize("kw", CONFIGS)
def test_export_round_trip_keeps_weights_and_tied_head(kw) -> None:
    cfg = nm.GPTConfig(**kw)
    torch.manual_seed(3)
    model = nm.GPTModel(cfg).to(torch.bfloat16)
    model._pack_block_weights()  # the fused path's weight layout must not change the export
    state = model.state_dict()
    _validate_like_export(state, cfg)
    buf = io.BytesIO()
    torch.save(state, buf)  # the reference's artifact writer (artifact.py:599)
    buf.seek(0)
    loaded = torch.load(buf, weights_only=True)
    _validate_like_export(loaded, cfg)
    fresh = nm.GPTModel(cfg).to(torch.bfloat16)
    fresh.load_state_dict(loaded, strict=True)
    assert (fresh.lm_head.weight is fresh.embedding.weight) == cfg.tie_embeddings
    for k, t in fresh.state_dict().items():
        assert torch.equal(t, state[k]), k


def test_oracle_state_loads_into_the_model() -> None:
    """A state written by the reference's module layout (the oracle's) loads strictly."""
    cfg = nm.GPTConfig(**CONFIGS[1])
    torch.manual_seed(0)
    oracle = R.OracleGPTModel(cfg)
    model = nm.GPTModel(cfg)
    model.load_state_dict(oracle.state_dict(), strict=True)
    for (k, a), (k2, b) in zip(sorted(model.state_dict().items()), sorted(oracle.state_dict().items())):
        assert k == k2 and torch.equal(a, b)


def test_metric_names_match_the_trainer() -> None:
    m = M.train_metrics(loss=2.5, learning_rate=3e-4, samples=16, tokens=8192, seconds=0.5, grad_norm=1.25)
    assert m == {"loss": 2.5, "learning_rate": 3e-4, "grad_norm": 1.25,
                 "samples_per_second": 32.0, "tokens_per_second": 16384.0}
    assert M.device_memory_metrics(torch.device("cpu")) == {}


def test_metric_history_line_schema() -> None:
    line = M.history_line(sequence=4, step=10, prefix=" train ",
                          metrics={"loss": float("nan"), "tokens_per_second": 1.5e5, "grad_norm": float("inf")},
                          consumed_samples=160, consumed_tokens=81920, data_shuffle_seed=1234,
                          recorded_at=12.5)
    rec = json.loads(line)
    assert rec == {
        "version": 1, "sequence": 4, "step": 10, "recorded_at": 12.5, "prefix": "train",
        "metrics": {"loss": "NaN", "tokens_per_second": 1.5e5, "grad_norm": "Infinity"},
        "trainer": {"consumed_samples": 160, "consumed_tokens": 81920},
        "data": {"epoch": 0, "sample_offset": 0, "shuffle_seed": 1234},
    }
    # compact, key-sorted, strict JSON as metric_history.py:182-190 writes it
    assert line == json.dumps(rec, separators=(",", ":"), sort_keys=True)
    assert list(json.loads(line)) == sorted(rec)
    with pytest.raises(ValueError):
        M.history_line(sequence=-1, step=0, prefix="train", metrics={}, consumed_samples=0, consumed_tokens=0)
    with pytest.raises(ValueError):
        M.history_line(sequence=0, step=0, prefix=" ", metrics={}, consumed_samples=0, consumed_tokens=0)
    with pytest.raises(TypeError):
        M.history_line(sequence=0, step=0, prefix="train", metrics={"loss": True}, consumed_samples=0,
                       consumed_tokens=0)
    assert math.isnan(float(json.loads(line)["metrics"]["loss"]))
