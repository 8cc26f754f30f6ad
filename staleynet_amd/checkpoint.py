"""Checkpoints of the reference's model, and the GEMM path's operands in them.

The format (crates/staleynet-model/src/checkpoint.rs:1-3, :60-96, :167):

* ``model.json``: the model configuration, the tensor manifest (name and value count of every
  parameter, in visitor order), the optimiser step, whether AdamW moments follow, and free-form
  training provenance;
* ``tensors.bin``: little-endian ``f32`` values, the parameters in visitor order, then (when
  ``has_optimizer_state``) every first moment and every second moment in the same order.

Visitor order (gpt.rs:91-101 and each layer's ``visit_parameters``): ``token_embedding``,
``position_embedding``, then per block ``attention_norm.gain``, ``attention.qkv.{weight,bias}``,
``attention.output.{weight,bias}``, ``feed_forward_norm.gain``,
``feed_forward.expand.{weight,bias}``, ``feed_forward.project.{weight,bias}``, then
``final_norm.gain`` and ``head.{weight,bias}``. A Linear's weight is ``[inputs, outputs]`` and
its bias ``[outputs]`` (layers/linear.rs:20-28), so a weight feeds ``Gpu::matmul`` as the right
operand of ``MatmulSpec::new(tokens, outputs, inputs)`` unchanged.

This module reads and writes the format (files written under a ``.partial`` name, then
renamed, as the reference does) and uploads the Linear layers' weights and biases as device
tensors. The embeddings and norm gains are read and checked but feed kernels outside the GEMM
path.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field
from typing import Any

import numpy as np

METADATA_FILE = "model.json"   # checkpoint.rs:18
TENSOR_FILE = "tensors.bin"    # checkpoint.rs:21
TEXT_VOCABULARY = 256 + 3      # vocabulary.rs:44: byte values plus three markers


@dataclass
class ModelConfig:
    """The fields of ``ModelConfig`` (crates/staleynet-model/src/config.rs) the manifest depends on;
    ``lyrics_bytes`` and ``lyric_cursor`` default as older metadata has them."""

    width: int
    heads: int
    layers: int
    feed_forward_multiplier: int
    context_length: int
    prompt_bytes: int
    codebooks: int
    codebook_size: int
    lyrics_bytes: int = 0
    lyric_cursor: bool = False
    extra: dict = field(default_factory=dict)

    @staticmethod
    def from_json(value: dict) -> "ModelConfig":
        known = {k: value[k] for k in ("width", "heads", "layers", "feed_forward_multiplier", "context_length",
                                       "prompt_bytes", "codebooks", "codebook_size") if k in value}
        config = ModelConfig(**known, lyrics_bytes=value.get("lyrics_bytes", 0),
                             lyric_cursor=value.get("lyric_cursor", False))
        config.extra = {k: v for k, v in value.items() if k not in known and k not in ("lyrics_bytes", "lyric_cursor")}
        return config

    def to_json(self) -> dict:
        out = {"width": self.width, "heads": self.heads, "layers": self.layers,
               "feed_forward_multiplier": self.feed_forward_multiplier, "context_length": self.context_length,
               "prompt_bytes": self.prompt_bytes, "lyrics_bytes": self.lyrics_bytes,
               "lyric_cursor": self.lyric_cursor, "codebooks": self.codebooks, "codebook_size": self.codebook_size}
        out.update(self.extra)
        return out

    def feed_forward_width(self) -> int:   # config.rs:78-80
        return self.width * self.feed_forward_multiplier

    def sequence_capacity(self) -> int:    # config.rs:84-86
        return self.context_length + self.lyrics_bytes

    def logits_width(self) -> int:         # config.rs:95-97
        return self.codebooks * self.codebook_size

    def vocabulary_size(self) -> int:      # vocabulary.rs:130-132
        return TEXT_VOCABULARY + self.codebooks * self.codebook_size


@dataclass(frozen=True)
class TensorEntry:
    """``TensorEntry`` (checkpoint.rs:25-33): a parameter's name and value count."""

    name: str
    len: int


@dataclass
class CheckpointMetadata:
    """``CheckpointMetadata`` (checkpoint.rs:36-53), the contents of ``model.json``."""

    model: ModelConfig
    tensors: list[TensorEntry]
    step: int
    has_optimizer_state: bool
    training: Any

    @staticmethod
    def from_json(value: dict) -> "CheckpointMetadata":
        return CheckpointMetadata(ModelConfig.from_json(value["model"]),
                                  [TensorEntry(t["name"], int(t["len"])) for t in value["tensors"]],
                                  int(value["step"]), bool(value["has_optimizer_state"]), value.get("training", {}))

    def to_json(self) -> dict:
        return {"model": self.model.to_json(), "tensors": [{"name": t.name, "len": t.len} for t in self.tensors],
                "step": self.step, "has_optimizer_state": self.has_optimizer_state, "training": self.training}


def parameter_shapes(config: ModelConfig) -> list[tuple[str, tuple[int, int]]]:
    """Every parameter of ``Gpt::new(config)`` (gpt.rs:42-75) as (name, (rows, cols)), in visitor order."""
    d, f = config.width, config.feed_forward_width()
    shapes = [("token_embedding", (config.vocabulary_size(), d)),
              ("position_embedding", (config.sequence_capacity(), d))]
    for i in range(config.layers):
        b = f"blocks.{i}"
        shapes += [(f"{b}.attention_norm.gain", (1, d)),
                   (f"{b}.attention.qkv.weight", (d, 3 * d)), (f"{b}.attention.qkv.bias", (1, 3 * d)),
                   (f"{b}.attention.output.weight", (d, d)), (f"{b}.attention.output.bias", (1, d)),
                   (f"{b}.feed_forward_norm.gain", (1, d)),
                   (f"{b}.feed_forward.expand.weight", (d, f)), (f"{b}.feed_forward.expand.bias", (1, f)),
                   (f"{b}.feed_forward.project.weight", (f, d)), (f"{b}.feed_forward.project.bias", (1, d))]
    shapes += [("final_norm.gain", (1, d)),
               ("head.weight", (d, config.logits_width())), ("head.bias", (1, config.logits_width()))]
    return shapes


def linear_layers(config: ModelConfig) -> list[str]:
    """The Linear layers (the GEMM path's products), in visitor order."""
    names = []
    for i in range(config.layers):
        names += [f"blocks.{i}.attention.qkv", f"blocks.{i}.attention.output",
                  f"blocks.{i}.feed_forward.expand", f"blocks.{i}.feed_forward.project"]
    return names + ["head"]


def read_metadata(directory: str) -> CheckpointMetadata:
    """``read_metadata`` (checkpoint.rs:158-163)."""
    with open(os.path.join(directory, METADATA_FILE)) as f:
        return CheckpointMetadata.from_json(json.load(f))


def read_values(directory: str) -> np.ndarray:
    """Every value of ``tensors.bin`` (little-endian f32; checkpoint.rs:214-228), memory-mapped."""
    path = os.path.join(directory, TENSOR_FILE)
    if os.path.getsize(path) == 0:
        return np.zeros(0, np.float32)
    return np.memmap(path, dtype="<f4", mode="r")


def stored_tensors(metadata: CheckpointMetadata, values: np.ndarray) -> dict[str, np.ndarray]:
    """The stored parameters by name, each a slice of ``values`` in file order (checkpoint.rs:231-242)."""
    stored, offset = {}, 0
    for entry in metadata.tensors:
        if offset + entry.len > len(values):
            raise ValueError("tensors.bin ends before every tensor was read")
        stored[entry.name] = values[offset:offset + entry.len]
        offset += entry.len
    return stored


def check_manifest(metadata: CheckpointMetadata) -> None:
    """``load``'s check (checkpoint.rs:171-186): the manifest must list the model's parameters, in
    visitor order, with their value counts."""
    expected = parameter_shapes(metadata.model)
    if len(metadata.tensors) < len(expected):
        raise ValueError("checkpoint has fewer tensors than the model")
    for entry, (name, (rows, cols)) in zip(metadata.tensors, expected):
        if entry.name != name or entry.len != rows * cols:
            raise ValueError(f"checkpoint tensor {entry.name} ({entry.len}) does not match parameter {name}")


def save(directory: str, config: ModelConfig, parameters: dict[str, np.ndarray], step: int = 0,
         training: Any = None, moments: tuple[list[np.ndarray], list[np.ndarray]] | None = None) -> None:
    """``save`` (checkpoint.rs:60-96): the parameters in visitor order (and the AdamW moments, every
    first then every second), each file written under ``.partial`` and renamed."""
    os.makedirs(directory, exist_ok=True)
    entries, blocks = [], []
    for name, (rows, cols) in parameter_shapes(config):
        value = np.ascontiguousarray(parameters[name], dtype="<f4").ravel()
        if value.size != rows * cols:
            raise ValueError(f"{name} has {value.size} values, the model {rows * cols}")
        entries.append(TensorEntry(name, value.size))
        blocks.append(value)
    if moments is not None:
        firsts, seconds = moments
        blocks += [np.ascontiguousarray(m, dtype="<f4").ravel() for m in list(firsts) + list(seconds)]
    _write_atomically(os.path.join(directory, TENSOR_FILE), lambda f: [f.write(b.tobytes()) for b in blocks])
    metadata = CheckpointMetadata(config, entries, step, moments is not None, {} if training is None else training)
    text = json.dumps(metadata.to_json(), indent=2)
    _write_atomically(os.path.join(directory, METADATA_FILE), lambda f: f.write(text.encode()))


def _write_atomically(path: str, write) -> None:
    """``write_atomically`` (checkpoint.rs:279-292)."""
    staging = path + ".partial"
    with open(staging, "wb") as f:
        write(f)
    os.replace(staging, path)


def load_linear_operands(gpu, directory: str) -> dict[str, tuple]:
    """Each Linear layer's weight ``[inputs, outputs]`` and bias ``[outputs]`` uploaded as device
    tensors, by layer name, after ``check_manifest``: the operands of ``Linear::forward``
    (``gpu.matmul_bias(MatmulSpec.new(tokens, outputs, inputs), x, weight, bias, y)``)."""
    from .gemm import Shape

    metadata = read_metadata(directory)
    check_manifest(metadata)
    stored = stored_tensors(metadata, read_values(directory))
    shapes = dict(parameter_shapes(metadata.model))
    operands = {}
    for layer in linear_layers(metadata.model):
        rows, cols = shapes[f"{layer}.weight"]
        weight = gpu.upload(Shape(rows, cols), np.asarray(stored[f"{layer}.weight"], dtype=np.float32))
        bias = gpu.upload(Shape.vector(cols), np.asarray(stored[f"{layer}.bias"], dtype=np.float32))
        operands[layer] = (weight, bias)
    return operands
