"""The oqpack.v1 container on the CPU: multi-shard round trip of LUT layers,
mmap access, tokenizer files, and the reference's integrity failure modes
(T/test_m1_oqpack_container.py:78-470: corrupt byte, missing shard,
unsupported version, tampered shape / dtype / size, missing tensor, missing
tokenizer file), on packages written by this build's writer."""
import json

import numpy as np
import pytest

from oracle import numpy_oracle as no


def make_weight(me, torch, r, rows, cols, block, bits, stages):
    G = (cols + block - 1) // block
    codes = r.integers(0, 1 << bits, size=(stages, rows * G))
    packed = np.stack([no.pack_codes(c, bits) for c in codes])
    return me.QuantizedWeight(
        original_shape=(rows, cols), block_size=block, bits_per_stage=bits,
        packed_codes=torch.from_numpy(packed.astype(np.uint8)),
        codebooks=torch.from_numpy(r.normal(size=(stages, 1 << bits, block)).astype(np.float32)),
        row_scales=torch.from_numpy(r.uniform(0.5, 1.5, size=rows).astype(np.float32)),
        metrics={})


@pytest.fixture
def package(pkg, tmp_path):
    import torch
    me, oq = pkg.math_engine, pkg.oqpack
    r = np.random.default_rng(0)
    layers = {"model.layers.0.mlp.up": make_weight(me, torch, r, 48, 40, 8, 4, 2),
              "model.layers.0.mlp.down": make_weight(me, torch, r, 40, 48, 16, 8, 1),
              "lm_head": make_weight(me, torch, r, 30, 32, 16, 2, 3)}
    biases = {"model.layers.0.mlp.up": torch.from_numpy(r.normal(size=48).astype(np.float32))}
    extra = {"model.norm.weight": torch.ones(40)}
    tok = tmp_path / "tok"
    tok.mkdir()
    (tok / "tokenizer.json").write_text('{"dummy": true}', encoding="utf-8")
    (tok / "tokenizer_config.json").write_text('{"bos_token": "<s>"}', encoding="utf-8")
    out = tmp_path / "pkg"
    manifest = oq.save_oqpack(layers, out, biases=biases, extra_tensors=extra, model_id="lut-test",
                              max_shard_bytes=2048, tokenizer_dir=tok, chat_template="{{ x }}")
    return dict(dir=out, manifest=manifest, layers=layers, biases=biases, extra=extra)


def test_roundtrip_multi_shard(pkg, package):
    import torch
    oq = pkg.oqpack
    m = package["manifest"]
    assert m.format_version == oq.OQPACK_FORMAT_VERSION == "oqpack.v1"
    assert len(m.shards) >= 2 and m.model_id == "lut-test"
    for i, shard in enumerate(m.shards):
        assert shard.filename == f"shard-{i + 1:05d}-of-{len(m.shards):05d}.safetensors"
    assert m.layer_specs["lm_head"]["codec"] == "adaptive_residual_vq"
    assert m.layer_specs["model.layers.0.mlp.up"]["has_bias"] is True
    assert set(m.tokenizer_files) == {"tokenizer.json", "tokenizer_config.json",
                                      "chat_template.jinja"}
    again = oq.verify_oqpack_integrity(package["dir"], verify_checksums=True)
    assert again.to_dict() == m.to_dict()
    tensors = oq.open_oqpack_mmap(package["dir"], verify_checksums=True)
    assert len(tensors) == len(m.tensors)
    for name, w in package["layers"].items():
        assert torch.equal(tensors[name + ".packed_codes"], w.packed_codes)
        assert torch.equal(tensors[name + ".codebooks"], w.codebooks)
        assert torch.equal(tensors[name + ".row_scales"], w.row_scales)
    layers, _ = oq.load_lut_layers(package["dir"], device="cpu")
    assert set(layers) == set(package["layers"])
    for name, w in package["layers"].items():
        got = layers[name].weight
        assert got.original_shape == w.original_shape and got.stages == w.stages
        assert torch.equal(got.packed_codes, w.packed_codes)
    assert torch.equal(layers["model.layers.0.mlp.up"].bias, package["biases"]["model.layers.0.mlp.up"])
    assert layers["lm_head"].bias is None


def _edit_manifest(d, fn):
    path = d / "oqpack_manifest.json"
    payload = json.loads(path.read_text(encoding="utf-8"))
    fn(payload)
    path.write_text(json.dumps(payload), encoding="utf-8")


def test_corrupt_shard_byte(pkg, package):
    d = package["dir"]
    path = d / package["manifest"].shards[0].filename
    data = bytearray(path.read_bytes())
    data[20] ^= 0xAA
    path.write_bytes(data)
    with pytest.raises(pkg.oqpack.OQPackValidationError) as e:
        pkg.oqpack.verify_oqpack_integrity(d, verify_checksums=True)
    assert "checksum mismatch" in str(e.value) or "Corrupt" in str(e.value)


def test_missing_shard(pkg, package):
    (package["dir"] / package["manifest"].shards[1].filename).unlink()
    with pytest.raises(pkg.oqpack.OQPackValidationError, match="(?i)missing"):
        pkg.oqpack.verify_oqpack_integrity(package["dir"])


@pytest.mark.parametrize("edit,msg", [
    (lambda p: p.__setitem__("format_version", "oqpack.v999"), "Unsupported format_version"),
    (lambda p: p["tensors"][next(iter(p["tensors"]))].__setitem__("shape", [999, 999]),
     "shape mismatch"),
    (lambda p: p["tensors"][next(iter(p["tensors"]))].__setitem__("dtype", "int8"),
     "dtype mismatch"),
    (lambda p: p["shards"][0].__setitem__("size_bytes", 123456789), "size mismatch"),
    (lambda p: p["tensors"].__setitem__("ghost.weight", dict(
        name="ghost.weight", shard=p["shards"][0]["filename"], dtype="float32", shape=[1],
        nbytes=4, role="other")), "missing from shards"),
    (lambda p: p.__setitem__("shards", []), "no shards"),
])
def test_tampered_manifest(pkg, package, edit, msg):
    _edit_manifest(package["dir"], edit)
    with pytest.raises(pkg.oqpack.OQPackValidationError, match=msg):
        pkg.oqpack.verify_oqpack_integrity(package["dir"])


def test_missing_tokenizer_file(pkg, package):
    (package["dir"] / "tokenizer.json").unlink()
    with pytest.raises(pkg.oqpack.OQPackValidationError, match="Tokenizer file missing"):
        pkg.oqpack.verify_oqpack_integrity(package["dir"])


def test_non_lut_layers_skipped_or_strict(pkg, package):
    oq = pkg.oqpack

    def add(p):
        p["layer_specs"]["experts"] = {"module_type": "fused_experts",
                                       "type": "residual_vq_fused_experts"}
    _edit_manifest(package["dir"], add)
    layers, _ = oq.load_lut_layers(package["dir"], device="cpu")
    assert "experts" not in layers and len(layers) == 3
    with pytest.raises(oq.OQPackValidationError, match="not a LUT layer"):
        oq.load_lut_layers(package["dir"], device="cpu", strict=True)


# --- a package written by the reference's own save_oqpack ---------------------------
# tests/golden/oqpack_ref_small/ and oqpack_ref_expected.npz come from
# tests/golden/make_oqpack_golden.py (the reference's quantize_model + save_oqpack,
# ojasx_24x96/oqpack.py:383-548, and its modules' forward outputs).

def _ref_package():
    import os
    from conftest import GOLDEN
    return os.path.join(GOLDEN, "oqpack_ref_small"), np.load(os.path.join(GOLDEN,
                                                                        "oqpack_ref_expected.npz"))


def test_reference_package_verifies_and_loads(pkg):
    """This build's verifier and reader accept the reference's package; the
    loaded layers through the NumPy oracle reproduce the reference modules'
    outputs (rel 1e-5)."""
    from conftest import rel_err
    oq = pkg.oqpack
    path, exp = _ref_package()
    m = oq.verify_oqpack_integrity(path)
    assert m.format_version == "oqpack.v1" and m.model_id == "ojasx-lut-interchange-fixture"
    assert sorted(m.layer_specs) == ["0", "2"]
    layers, _ = oq.load_lut_layers(path, device="cpu")
    assert [layers[k].weight.stages for k in ("0", "2")] == list(exp["stages"])
    for name, x, y in (("0", exp["x0"], exp["y0"]), ("2", exp["x2"], exp["y2"])):
        w, b = layers[name].weight, layers[name].bias
        rows, cols = w.original_shape
        got = no.subspace_lut_rvq_gemm(x, w.codebooks.numpy(), w.packed_codes.numpy(),
                                       w.bits_per_stage, rows, cols, w.block_size,
                                       w.row_scales.numpy(), None if b is None else b.numpy())
        assert rel_err(got, y) < 1e-5, name


def test_reference_package_tamper_detected(pkg, tmp_path):
    """A flipped byte in the reference's shard fails the checksum check."""
    import shutil
    oq = pkg.oqpack
    path, _ = _ref_package()
    bad = tmp_path / "bad"
    shutil.copytree(path, bad)
    shard = next(bad.glob("shard-*.safetensors"))
    data = bytearray(shard.read_bytes())
    data[-5] ^= 0x40
    shard.write_bytes(bytes(data))
    with pytest.raises(oq.OQPackValidationError):
        oq.verify_oqpack_integrity(bad)


def test_reference_reads_our_package():
    """Recorded at fixture generation: the reference's
    load_quantized_model_from_oqpack (ojasx_24x96/oqpack.py:688-754) read the
    package this build's save_oqpack wrote from the same layers, and its
    modules gave the reference package's outputs bit for bit."""
    _, exp = _ref_package()
    assert np.array_equal(exp["ours_by_ref_y0"], exp["y0"])
    assert np.array_equal(exp["ours_by_ref_y2"], exp["y2"])
