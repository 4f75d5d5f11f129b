"""Training-step metrics in the reference's names and JSONL history format.

The reference's trainer reports, per logged step, ``loss``, ``grad_norm``,
``learning_rate``, ``samples_per_second``, ``tokens_per_second`` and four device
memory figures (training/trainer.py:449-455, 613-624, 752-776), and appends
each record to a versioned JSONL history (training/metric_history.py:13-19,
40-45, 161-190).  ``train_metrics`` computes the same names for this
package's step; ``history_line`` writes one record in the same schema, so the
reference's history reader accepts the file.
"""

from __future__ import annotations

import json
import math
import time
from typing import Mapping

import torch

METRIC_HISTORY_VERSION = 1

_GIB = float(1 << 30)


def device_memory_metrics(device: torch.device) -> dict[str, float]:
    """The four memory figures of trainer.py:752-776 (GiB) for a CUDA/HIP device."""
    if device.type != "cuda":
        return {}
    return {
        "gpu_memory_allocated_gib": torch.cuda.memory_allocated(device) / _GIB,
        "gpu_peak_memory_allocated_gib": torch.cuda.max_memory_allocated(device) / _GIB,
        "gpu_memory_reserved_gib": torch.cuda.memory_reserved(device) / _GIB,
        "gpu_peak_memory_reserved_gib": torch.cuda.max_memory_reserved(device) / _GIB,
    }


def train_metrics(*, loss: float, learning_rate: float, samples: int, tokens: int, seconds: float,
                  grad_norm: float | None = None, device: torch.device | None = None) -> dict[str, float]:
    """Metrics of ``samples`` samples / ``tokens`` tokens trained in ``seconds``
    (trainer.py:449-455 and 613-624: rates over the logging interval)."""
    elapsed = max(float(seconds), 1.0e-12)
    out = {"loss": float(loss), "learning_rate": float(learning_rate)}
    if grad_norm is not None:
        out["grad_norm"] = float(grad_norm)
    out["samples_per_second"] = samples / elapsed
    out["tokens_per_second"] = tokens / elapsed
    if device is not None:
        out.update(device_memory_metrics(device))
    return out


def _encode(value: float) -> float | str:
    # metric_history.py:40-47: non-finite values as strings, JSON has no NaN
    if math.isnan(value):
        return "NaN"
    if value == float("inf"):
        return "Infinity"
    if value == float("-inf"):
        return "-Infinity"
    return value


def _count(name: str, value: int | None, optional: bool = False) -> int | None:
    if value is None and optional:
        return None
    if isinstance(value, bool) or not isinstance(value, int) or value < 0:
        raise ValueError(f"{name} must be a non-negative integer")
    return value


def history_line(*, sequence: int, step: int, prefix: str, metrics: Mapping[str, float],
                 consumed_samples: int, consumed_tokens: int, data_epoch: int = 0,
                 data_sample_offset: int = 0, data_shuffle_seed: int | None = None,
                 recorded_at: float | None = None) -> str:
    """One metric-history record as the reference writes it
    (MetricHistoryRecord.to_dict / to_json_line, metric_history.py:161-190)."""
    if not isinstance(prefix, str) or not prefix.strip():
        raise ValueError("metric prefix must be a non-empty string")
    values = {}
    for name, value in metrics.items():
        if isinstance(value, bool) or not isinstance(value, (int, float)):
            raise TypeError(f"metric {name!r} must be numeric")
        values[str(name)] = _encode(float(value))
    record = {
        "version": METRIC_HISTORY_VERSION,
        "sequence": _count("metric sequence", sequence),
        "step": _count("metric step", step),
        "recorded_at": time.time() if recorded_at is None else float(recorded_at),
        "prefix": prefix.strip(),
        "metrics": values,
        "trainer": {
            "consumed_samples": _count("consumed_samples", consumed_samples),
            "consumed_tokens": _count("consumed_tokens", consumed_tokens),
        },
        "data": {
            "epoch": _count("data_epoch", data_epoch),
            "sample_offset": _count("data_sample_offset", data_sample_offset),
            "shuffle_seed": _count("data_shuffle_seed", data_shuffle_seed, optional=True),
        },
    }
    return json.dumps(record, ensure_ascii=False, separators=(",", ":"), sort_keys=True, allow_nan=False)
