"""The checkpoint format (crates/staleynet-model/src/checkpoint.rs) and the GEMM operands in it.

CPU: the manifest restatement (visitor order and value counts, gpt.rs:42-101) against three
``best-model.json`` files the reference's runs wrote (tests/golden/checkpoints: smoke, lyrics-orin
with a lyrics field, pq-large with 16 codebooks); the reference's own checkpoint unit tests
(checkpoint.rs:296-348); save/read round trips, the byte order and the optimiser moments' order;
the load checks. GPU: a Linear forward from weights read back out of a saved checkpoint, against
the oracle.
"""
import json
import os

import numpy as np
import pytest

from staleynet_amd import checkpoint as ck

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "checkpoints")
RUNS = ["smoke", "lyrics-orin", "pq-large"]


def golden(run):
    with open(os.path.join(GOLDEN, f"{run}.json")) as f:
        return ck.CheckpointMetadata.from_json(json.load(f))


@pytest.mark.parametrize("run", RUNS)
def test_manifest_restatement_matches_the_reference_runs(run):
    metadata = golden(run)
    expected = [(name, rows * cols) for name, (rows, cols) in ck.parameter_shapes(metadata.model)]
    assert [(t.name, t.len) for t in metadata.tensors] == expected
    ck.check_manifest(metadata)


def test_reference_tensor_entry_and_metadata_round_trip_json():
    # checkpoint.rs:300-327
    entry = ck.TensorEntry("blocks.0.attention.qkv.weight", 196_608)
    assert ck.TensorEntry(**json.loads(json.dumps(entry.__dict__))) == entry
    metadata = ck.CheckpointMetadata(ck.ModelConfig(256, 8, 6, 4, 768, 126, 4, 1024),
                                     [ck.TensorEntry("token_embedding", 1_114_880)], 7, False,
                                     {"seed": 1, "batch_size": 4})
    decoded = ck.CheckpointMetadata.from_json(json.loads(json.dumps(metadata.to_json())))
    assert decoded.model == metadata.model and decoded.tensors == metadata.tensors
    assert decoded.step == 7 and decoded.has_optimizer_state is False and decoded.training == metadata.training


def test_reference_older_metadata_defaults_the_lyrics_field_to_zero():
    # checkpoint.rs:329-347
    encoded = {"model": {"width": 256, "heads": 8, "layers": 6, "feed_forward_multiplier": 4,
                         "context_length": 768, "prompt_bytes": 126, "codebooks": 4, "codebook_size": 1024},
               "tensors": [], "step": 0, "has_optimizer_state": False, "training": {}}
    decoded = ck.CheckpointMetadata.from_json(encoded)
    assert decoded.model.lyrics_bytes == 0 and decoded.step == 0


def small_config():
    return ck.ModelConfig(width=64, heads=4, layers=2, feed_forward_multiplier=4, context_length=32, prompt_bytes=8,
                          codebooks=2, codebook_size=16)


def random_parameters(config, seed=0):
    rng = np.random.default_rng(seed)
    return {name: rng.normal(0, 0.02, rows * cols).astype(np.float32)
            for name, (rows, cols) in ck.parameter_shapes(config)}


def test_save_then_read_round_trips_in_visitor_order(tmp_path):
    config = small_config()
    params = random_parameters(config)
    ck.save(str(tmp_path), config, params, step=42, training={"seed": 3})
    assert not any(name.endswith(".partial") for name in os.listdir(tmp_path))
    metadata = ck.read_metadata(str(tmp_path))
    assert metadata.step == 42 and metadata.has_optimizer_state is False and metadata.training == {"seed": 3}
    ck.check_manifest(metadata)
    stored = ck.stored_tensors(metadata, ck.read_values(str(tmp_path)))
    for name, value in params.items():
        assert np.array_equal(stored[name], value)
    # Little-endian f32, the parameters back to back.
    total = sum(v.size for v in params.values())
    assert os.path.getsize(tmp_path / ck.TENSOR_FILE) == 4 * total
    first = params["token_embedding"][0]
    assert (tmp_path / ck.TENSOR_FILE).read_bytes()[:4] == np.array([first], "<f4").tobytes()


def test_optimizer_moments_follow_the_parameters_firsts_then_seconds(tmp_path):
    config = small_config()
    params = random_parameters(config)
    firsts = [np.full(v.size, 1.0, np.float32) for v in params.values()]
    seconds = [np.full(v.size, 2.0, np.float32) for v in params.values()]
    ck.save(str(tmp_path), config, params, moments=(firsts, seconds))
    metadata = ck.read_metadata(str(tmp_path))
    values = np.asarray(ck.read_values(str(tmp_path)))
    n = sum(v.size for v in params.values())
    assert metadata.has_optimizer_state and values.size == 3 * n
    assert np.all(values[n:2 * n] == 1.0) and np.all(values[2 * n:] == 2.0)


def test_load_checks_raise_the_reference_messages(tmp_path):
    config = small_config()
    ck.save(str(tmp_path), config, random_parameters(config))
    metadata = ck.read_metadata(str(tmp_path))
    wrong = ck.CheckpointMetadata(metadata.model, [ck.TensorEntry(metadata.tensors[0].name, 5)] + metadata.tensors[1:],
                                  0, False, {})
    with pytest.raises(ValueError, match="does not match parameter token_embedding"):
        ck.check_manifest(wrong)
    short = ck.CheckpointMetadata(metadata.model, metadata.tensors[:-1], 0, False, {})
    with pytest.raises(ValueError, match="fewer tensors than the model"):
        ck.check_manifest(short)
    with pytest.raises(ValueError, match="ends before every tensor"):
        ck.stored_tensors(metadata, np.zeros(10, np.float32))


@pytest.mark.gpu
def test_linear_forward_from_checkpoint_weights_matches_the_oracle(gpu, tmp_path):
    # Linear::forward (linear.rs:43-48) with block 0's qkv and the head read back from a saved
    # checkpoint: matmul_bias against the oracle's matmul + add_row_bias.
    from oracle import oracle
    from staleynet_amd.gemm import MatmulSpec, Shape

    config = small_config()
    params = random_parameters(config, seed=1)
    ck.save(str(tmp_path), config, params)
    operands = ck.load_linear_operands(gpu, str(tmp_path))
    assert list(operands) == ck.linear_layers(config)
    tokens = 96
    x = np.random.default_rng(2).normal(0, 1, tokens * config.width).astype(np.float32)
    X = gpu.upload(Shape(tokens, config.width), x)
    for layer in ("blocks.0.attention.qkv", "head"):
        weight, bias = operands[layer]
        outputs = weight.shape().cols
        y = gpu.zeros(Shape(tokens, outputs))
        gpu.matmul_bias(MatmulSpec.new(tokens, outputs, config.width), X, weight, bias, y)
        expected = np.zeros(tokens * outputs, np.float32)
        oracle.matmul(oracle.Product(tokens, outputs, config.width), x, params[f"{layer}.weight"], expected)
        oracle.add_row_bias(expected, outputs, params[f"{layer}.bias"])
        assert oracle.relative_error(expected, gpu.download(y)) < 1e-5
