"""The C++ host layer (decisive_amd/host): the reference's inference API
restated over the C ABI, run as compiled test programs."""
import hashlib
import json
import os
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
HOST = ROOT / "decisive_amd" / "host"
BUILD = HOST / "build"


def _program(name: str) -> Path:
    """The test program, rebuilt by make when a source or header changed."""
    exe = BUILD / name
    subprocess.run(["make", "-s", "-C", str(HOST), str(exe)], check=True)
    return exe


def _run(exe: Path, timeout: int, env=None):
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=timeout,
                       env={**os.environ, **(env or {})})
    print(r.stdout)
    print(r.stderr)
    return r


REVISION = "6d771ad7b5ecff5e93b8fc7b90d4c5ccc341954d"
HIDDEN, VOCAB, LAYERS = 2560, 50, 32


def write_checkpoint(root: Path, oracle) -> Path:
    """A complete q4-e4 packed checkpoint in the layout export_packed.rs:13-103
    writes and prepare_hf_q4.py:71-114 validates (the reference's own test
    builds the same layout, test_prepare_hf_q4.py:13-45), with real packed
    data: per layer a [4 x 128] matrix (packed) and a [128] vector (BF16),
    an embedding [50 x 2560], the readout [255 x 2560] and the final norm.
    Digests come from hashlib, independent of the library's SHA-256."""
    rng = np.random.default_rng(11)
    root.mkdir(parents=True, exist_ok=True)
    files, layers, shard0, shard1 = {}, [], {}, {}

    def bf16(values):
        return oracle.f32_to_bf16(values.astype(np.float32))

    def write(name, data: bytes):
        (root / name).write_bytes(data)
        files[name] = {"bytes": len(data), "sha256": hashlib.sha256(data).hexdigest()}

    offset = 0
    for layer in range(LAYERS):
        mat = f"language_model.layers.{layer}.mlp.weight"
        vec = f"language_model.layers.{layer}.norm.weight"
        shard0[mat] = {"dtype": "BF16", "shape": [4, 128], "data_offsets": [offset, offset + 1024]}
        shard0[vec] = {"dtype": "BF16", "shape": [128], "data_offsets": [offset + 1024, offset + 1280]}
        offset += 1280
        packed = oracle.pack_g64(bf16(rng.standard_normal((4, 128)) * 0.02), 4, 128, 4).tobytes()
        raw = bf16(rng.standard_normal(128) * 0.1).tobytes()
        name = f"q4-e4-layer-{layer:02}.bin"
        write(name, packed + raw)
        layers.append({"file": name, "bytes": len(packed) + len(raw), "tensors": [
            {"name": mat, "shape": [4, 128], "start": 0, "end": len(packed)},
            {"name": vec, "shape": [128], "start": len(packed), "end": len(packed) + len(raw)}]})
    shard0["language_model.embed_tokens.weight"] = {"dtype": "BF16", "shape": [VOCAB, HIDDEN],
                                                    "data_offsets": [offset, offset + VOCAB * HIDDEN * 2]}
    shard1["language_model.norm.weight"] = {"dtype": "BF16", "shape": [HIDDEN], "data_offsets": [0, HIDDEN * 2]}
    shard1["__metadata__"] = {"format": "pt"}
    write("q4-e4-embedding.bin", oracle.pack_g64(bf16(rng.standard_normal((VOCAB, HIDDEN))), VOCAB, HIDDEN, 4).tobytes())
    write("q4-e4-readout.bin", oracle.pack_g64(bf16(rng.standard_normal((255, HIDDEN)) * 0.02), 255, HIDDEN, 4).tobytes())
    write("q4-e4-norm.bin", bf16(rng.standard_normal(HIDDEN) * 0.1).tobytes())
    manifest = {"schema_version": 1, "revision": REVISION, "scheme": "q4-w4a8-e4-r4-g64", "group_size": 64,
                "group_bytes": 36, "embedding_row_bytes": HIDDEN // 64 * 36, "layers": layers,
                "headers": [json.dumps(shard0), json.dumps(shard1)], "embedding": "q4-e4-embedding.bin",
                "readout": "q4-e4-readout.bin", "norm": "q4-e4-norm.bin",
                "decoder_bytes": sum(l["bytes"] for l in layers), "files": dict(sorted(files.items()))}
    (root / "packed-q4-e4.json").write_text(json.dumps(manifest, indent=2))
    (root / "decision_config.json").write_text(json.dumps({"temperature": 1.5539091673122623}))
    return root


PPLX_SMALL = dict(layers=4, hidden=256, ff=512, delta_heads=4, delta_key_heads=2, delta_head_dim=128,
                  attn_heads=4, attn_kv_heads=2, attn_head_dim=256)


def write_pplx_checkpoint(root: Path, oracle) -> Path:
    """The random Pplx decider of tests/pplx_model.py (PPLX_SMALL, 64-token
    vocabulary) as a q4-e4 packed checkpoint (export_packed.rs:13-103 layout),
    plus expected_logits.json: the oracle's logits for one chunk."""
    from tests import pplx_model
    model = pplx_model.random_model(oracle, PPLX_SMALL, seed=5)
    root.mkdir(parents=True, exist_ok=True)
    files, layers, shard0, shard1 = {}, [], {}, {}

    def write(name, data: bytes):
        (root / name).write_bytes(data)
        files[name] = {"bytes": len(data), "sha256": hashlib.sha256(data).hexdigest()}

    def bf16_bytes(values):
        return oracle.f32_to_bf16(np.asarray(values, np.float32)).tobytes()

    cw = pplx_model.conv_width(PPLX_SMALL)
    offset = 0
    for i in range(PPLX_SMALL["layers"]):
        prefix = f"language_model.layers.{i}."
        blob, tensors = b"", []
        for name in sorted(n for n in list(model.packed) + list(model.vectors) if n.startswith(prefix)):
            if name in model.packed:
                wire, rows, cols = model.packed[name]
                data, shape = wire.tobytes(), [rows, cols]
            else:
                values = model.vectors[name]
                data = bf16_bytes(values)
                shape = [cw, 1, 4] if name.endswith("conv1d.weight") else [values.size]
            n_el = int(np.prod(shape))
            shard0[name] = {"dtype": "BF16", "shape": shape, "data_offsets": [offset, offset + 2 * n_el]}
            offset += 2 * n_el
            tensors.append({"name": name, "shape": shape, "start": len(blob), "end": len(blob) + len(data)})
            blob += data
        fname = f"q4-e4-layer-{i:02}.bin"
        write(fname, blob)
        layers.append({"file": fname, "bytes": len(blob), "tensors": tensors})
    vocab = model.embedding.shape[0]
    shard0["language_model.embed_tokens.weight"] = {"dtype": "BF16", "shape": [vocab, 256],
                                                    "data_offsets": [offset, offset + vocab * 512]}
    shard1["language_model.norm.weight"] = {"dtype": "BF16", "shape": [256], "data_offsets": [0, 512]}
    write("q4-e4-embedding.bin", model.embedding.tobytes())
    write("q4-e4-readout.bin", model.packed["readout"][0].tobytes())
    write("q4-e4-norm.bin", bf16_bytes(model.vectors["language_model.norm.weight"]))
    manifest = {"schema_version": 1, "revision": REVISION, "scheme": "q4-w4a8-e4-r4-g64", "group_size": 64,
                "group_bytes": 36, "embedding_row_bytes": 256 // 64 * 36, "layers": layers,
                "headers": [json.dumps(shard0), json.dumps(shard1)], "embedding": "q4-e4-embedding.bin",
                "readout": "q4-e4-readout.bin", "norm": "q4-e4-norm.bin",
                "decoder_bytes": sum(l["bytes"] for l in layers), "files": dict(sorted(files.items()))}
    (root / "packed-q4-e4.json").write_text(json.dumps(manifest, indent=2))
    (root / "decision_config.json").write_text(json.dumps({"temperature": 1.5539091673122623}))
    ids = [int(v) for v in np.random.default_rng(9).integers(0, vocab, 40)]
    markers = [39, 7, 20]
    logits = pplx_model.ref_forward(oracle, model, np.array(ids), markers)
    (root / "expected_logits.json").write_text(json.dumps({"ids": ids, "markers": markers,
                                                           "logits": logits.tolist()}))
    return root


def test_model_cache_parameters_and_embedding_cache_on_cpu(tmp_path, oracle):
    """Ports of src/inference/tests.rs:57-141 plus EmbeddingCache
    (browser/pplx.rs:45-138), error-code mapping (mod.rs:56-78), the answer
    step (input.rs) and the packed checkpoint reader (prepare_hf_q4.py)."""
    ck = write_checkpoint(tmp_path / "ck", oracle)
    pk = write_pplx_checkpoint(tmp_path / "pplx", oracle)
    r = _run(_program("test_inference"), 120, {"DZ_CHECKPOINT_DIR": str(ck), "DZ_PPLX_CHECKPOINT_DIR": str(pk)})
    assert r.returncode == 0, r.stderr
    assert "0 failed check(s)" in r.stdout


@pytest.mark.gpu
def test_rocm_backend_behind_model(tmp_path, oracle):
    """Model<Rocm> on the GPU: predictions equal the direct encoder forward bit
    for bit, cache reuse, splitting by maxSequenceTokens, failure clearing,
    answers, and a backend opened on a packed checkpoint."""
    ck = write_checkpoint(tmp_path / "ck", oracle)
    pk = write_pplx_checkpoint(tmp_path / "pplx", oracle)
    r = _run(_program("test_rocm_backend"), 240, {"DZ_CHECKPOINT_DIR": str(ck), "DZ_PPLX_CHECKPOINT_DIR": str(pk)})
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failed check(s)" in r.stdout
