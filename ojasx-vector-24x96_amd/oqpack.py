"""The reference's on-disk container (oqpack.v1) for the LUT path: read,
verify and write packages, and load their residual-VQ linear layers onto the
GPU as math-engine weights or, for single-stage 8-bit block-16 layers, as the
tiled LUT-GEMV handles.

Container (ojasx_24x96/oqpack.py:36-160, 383-548, 551-685): a JSON manifest
``oqpack_manifest.json`` (format ``oqpack.v1``) listing safetensors shards
``shard-NNNNN-of-MMMMM.safetensors`` with their sha256 and size, every tensor's
shard, dtype, shape, byte count and role, and per-layer specs; an
``adaptive_residual_vq`` linear (ojasx_24x96/module.py:116-219) stores
``<layer>.packed_codes`` [stages, ceil(rows * G * bits / 8)] uint8,
``<layer>.codebooks`` [stages, 2^bits, block] fp32, ``<layer>.row_scales``
[rows] fp32 and, with a bias, ``<layer>.bias``.  Manifest, verification and
error messages follow the reference so its packages and ours are
interchangeable; tensors are read with safetensors (no pickle).
"""
from __future__ import annotations

import hashlib
import json
import shutil
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Dict, List, Optional, Tuple, Union

OQPACK_FORMAT_VERSION = "oqpack.v1"
MANIFEST_FILENAME = "oqpack_manifest.json"
CODEC_SCHEMA_VERSION = "ojasx-24x96-v1.0"
_TOKENIZER_FILES = ("tokenizer.json", "tokenizer_config.json", "special_tokens_map.json",
                    "chat_template.jinja", "vocab.json", "merges.txt")


class OQPackValidationError(ValueError):
    """A package fails integrity, checksum or schema validation."""


@dataclass(frozen=True)
class OQPackShardEntry:
    filename: str
    sha256: str
    size_bytes: int
    tensor_names: Tuple[str, ...]

    def to_dict(self) -> Dict[str, Any]:
        return {"filename": self.filename, "sha256": self.sha256, "size_bytes": self.size_bytes,
                "tensor_names": list(self.tensor_names)}

    @classmethod
    def from_dict(cls, d: Dict[str, Any]) -> "OQPackShardEntry":
        return cls(str(d["filename"]), str(d["sha256"]), int(d["size_bytes"]),
                   tuple(d.get("tensor_names", ())))


@dataclass(frozen=True)
class OQPackTensorRecord:
    name: str
    shard: str
    dtype: str
    shape: Tuple[int, ...]
    nbytes: int
    role: str

    def to_dict(self) -> Dict[str, Any]:
        return {"name": self.name, "shard": self.shard, "dtype": self.dtype,
                "shape": list(self.shape), "nbytes": self.nbytes, "role": self.role}

    @classmethod
    def from_dict(cls, d: Dict[str, Any]) -> "OQPackTensorRecord":
        return cls(str(d["name"]), str(d["shard"]), str(d["dtype"]), tuple(d.get("shape", ())),
                   int(d["nbytes"]), str(d.get("role", "other")))


@dataclass
class OQPackManifest:
    format_version: str
    codec_schema_version: str
    model_id: str
    source_checkpoint_sha256: str
    architecture_profile: Dict[str, object]
    memory_admission: Dict[str, object]
    quantization_plan: Dict[str, object]
    quality_certificate: Optional[Dict[str, object]]
    shards: List[OQPackShardEntry]
    tensors: Dict[str, OQPackTensorRecord]
    layer_specs: Dict[str, Dict[str, object]]
    tokenizer_files: List[str]
    chat_template: Optional[str]

    def to_dict(self) -> Dict[str, Any]:
        return {
            "format_version": self.format_version,
            "codec_schema_version": self.codec_schema_version,
            "model_id": self.model_id,
            "source_checkpoint_sha256": self.source_checkpoint_sha256,
            "architecture_profile": self.architecture_profile,
            "memory_admission": self.memory_admission,
            "quantization_plan": self.quantization_plan,
            "quality_certificate": self.quality_certificate,
            "shards": [s.to_dict() for s in self.shards],
            "tensors": {k: v.to_dict() for k, v in self.tensors.items()},
            "layer_specs": self.layer_specs,
            "tokenizer_files": list(self.tokenizer_files),
            "chat_template": self.chat_template,
        }

    @classmethod
    def from_dict(cls, d: Dict[str, Any]) -> "OQPackManifest":
        return cls(
            format_version=str(d.get("format_version", "")),
            codec_schema_version=str(d.get("codec_schema_version", "")),
            model_id=str(d.get("model_id", "unknown")),
            source_checkpoint_sha256=str(d.get("source_checkpoint_sha256", "")),
            architecture_profile=dict(d.get("architecture_profile", {})),
            memory_admission=dict(d.get("memory_admission", {})),
            quantization_plan=dict(d.get("quantization_plan", {})),
            quality_certificate=d.get("quality_certificate"),
            shards=[OQPackShardEntry.from_dict(s) for s in d.get("shards", [])],
            tensors={k: OQPackTensorRecord.from_dict(v) for k, v in d.get("tensors", {}).items()},
            layer_specs=dict(d.get("layer_specs", {})),
            tokenizer_files=list(d.get("tokenizer_files", [])),
            chat_template=d.get("chat_template"),
        )


def _sha256(path: Path) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        while True:
            chunk = f.read(1 << 20)
            if not chunk:
                break
            h.update(chunk)
    return h.hexdigest()


def _dtype_name(t) -> str:
    return str(t.dtype).replace("torch.", "")


def verify_oqpack_integrity(package_dir: Union[str, Path], *,
                            verify_checksums: bool = True) -> OQPackManifest:
    """Checks of ojasx_24x96/oqpack.py:551-665: manifest present and parsable,
    format version, every shard present with its recorded size (and sha256),
    tensor names per shard, no duplicates, every tensor's shard, shape, dtype
    and byte count, no declared tensor missing, tokenizer files present."""
    from safetensors import SafetensorError, safe_open
    pkg = Path(package_dir)
    if not pkg.is_dir():
        raise OQPackValidationError(f"OQPack directory does not exist: {pkg}")
    manifest_path = pkg / MANIFEST_FILENAME
    if not manifest_path.is_file():
        raise OQPackValidationError(f"Missing manifest file: {manifest_path}")
    try:
        data = json.loads(manifest_path.read_text(encoding="utf-8"))
    except Exception as e:
        raise OQPackValidationError(f"Corrupt manifest JSON: {e}") from e
    manifest = OQPackManifest.from_dict(data)
    if manifest.format_version != OQPACK_FORMAT_VERSION:
        raise OQPackValidationError(f"Unsupported format_version {manifest.format_version!r}, "
                                    f"expected {OQPACK_FORMAT_VERSION!r}")
    if not manifest.shards:
        raise OQPackValidationError("OQPack manifest specifies no shards")
    seen = set()
    for shard in manifest.shards:
        path = pkg / shard.filename
        if not path.is_file():
            raise OQPackValidationError(f"Shard file missing: {shard.filename}")
        size = path.stat().st_size
        if size != shard.size_bytes:
            raise OQPackValidationError(f"Shard {shard.filename} size mismatch: expected "
                                        f"{shard.size_bytes}, found {size}")
        if verify_checksums:
            sha = _sha256(path)
            if sha != shard.sha256:
                raise OQPackValidationError(f"Shard {shard.filename} checksum mismatch: expected "
                                            f"{shard.sha256}, found {sha}")
        try:
            with safe_open(str(path), framework="pt", device="cpu") as handle:
                keys = set(handle.keys())
                want = set(shard.tensor_names)
                if keys != want:
                    raise OQPackValidationError(
                        f"Shard {shard.filename} tensor names mismatch. Missing: {want - keys}, "
                        f"Extra: {keys - want}")
                dups = seen & keys
                if dups:
                    raise OQPackValidationError(
                        f"Duplicate tensor names across shards: {dups} in {shard.filename}")
                seen |= keys
                for name in keys:
                    rec = manifest.tensors.get(name)
                    if rec is None:
                        raise OQPackValidationError(f"Tensor {name} in shard {shard.filename} not "
                                                    "found in manifest.tensors")
                    if rec.shard != shard.filename:
                        raise OQPackValidationError(f"Tensor {name} shard mismatch: record says "
                                                    f"{rec.shard}, found in {shard.filename}")
                    sl = handle.get_slice(name)
                    shape = tuple(sl.get_shape())
                    if shape != tuple(rec.shape):
                        raise OQPackValidationError(f"Tensor {name} shape mismatch: expected "
                                                    f"{rec.shape}, got {shape}")
                    t = handle.get_tensor(name)
                    if _dtype_name(t) != str(rec.dtype).replace("torch.", ""):
                        raise OQPackValidationError(f"Tensor {name} dtype mismatch: expected "
                                                    f"{rec.dtype}, got {_dtype_name(t)}")
                    if t.numel() * t.element_size() != rec.nbytes:
                        raise OQPackValidationError(
                            f"Tensor {name} nbytes mismatch: expected {rec.nbytes}, got "
                            f"{t.numel() * t.element_size()}")
        except SafetensorError as e:
            raise OQPackValidationError(f"Corrupt safetensors shard {shard.filename}: {e}") from e
        except OQPackValidationError:
            raise
        except Exception as e:
            raise OQPackValidationError(f"Error inspecting shard {shard.filename}: {e}") from e
    missing = set(manifest.tensors) - seen
    if missing:
        raise OQPackValidationError(
            f"Tensors declared in manifest.tensors missing from shards: {missing}")
    for tok in manifest.tokenizer_files:
        if not (pkg / tok).is_file():
            raise OQPackValidationError(f"Tokenizer file missing: {tok}")
    return manifest


def open_oqpack_mmap(package_dir: Union[str, Path], *, device: str = "cpu",
                     verify_checksums: bool = False):
    """Every tensor of the package (ojasx_24x96/oqpack.py:668-685), memory
    mapped by safetensors, after verification."""
    from safetensors import safe_open
    pkg = Path(package_dir)
    manifest = verify_oqpack_integrity(pkg, verify_checksums=verify_checksums)
    tensors = {}
    for shard in manifest.shards:
        with safe_open(str(pkg / shard.filename), framework="pt", device=device) as handle:
            for key in handle.keys():
                tensors[key] = handle.get_tensor(key)
    return tensors


def _linear_spec(w, has_bias: bool, source_dtype: str) -> Dict[str, object]:
    rows, cols = w.original_shape
    return {"module_type": "linear", "type": "residual_vq_linear", "codec": "adaptive_residual_vq",
            "in_features": cols, "out_features": rows, "block_size": w.block_size,
            "bits_per_stage": w.bits_per_stage, "stages": w.stages, "gain_bits": 0,
            "rotation_reflections": 0, "rotation_seed": 20261104, "adaptive_stages": True,
            "source_dtype": source_dtype, "has_bias": has_bias, "bias": has_bias,
            "active_counts": None}


def save_oqpack(layers: Dict[str, object], output_dir: Union[str, Path], *,
                biases: Optional[Dict[str, object]] = None,
                extra_tensors: Optional[Dict[str, object]] = None,
                roles: Optional[Dict[str, str]] = None, model_id: str = "unknown",
                source_checkpoint_sha256: str = "", max_shard_bytes: int = 512 * 1024 * 1024,
                tokenizer_dir: Optional[Union[str, Path]] = None,
                chat_template: Optional[str] = None,
                source_dtype: str = "float32") -> OQPackManifest:
    """Write LUT layers (name -> math_engine.QuantizedWeight, residual-VQ
    linears) and any extra dense tensors as an oqpack.v1 package, with the
    reference's shard split (tensors in order, a new shard when the next
    tensor would pass max_shard_bytes), naming, manifest and tokenizer files
    (ojasx_24x96/oqpack.py:383-548)."""
    import safetensors.torch
    out = Path(output_dir)
    out.mkdir(parents=True, exist_ok=True)
    biases = biases or {}
    roles = roles or {}
    sd: Dict[str, object] = {}
    specs: Dict[str, Dict[str, object]] = {}
    for name, w in layers.items():
        sd[f"{name}.packed_codes"] = w.packed_codes
        sd[f"{name}.codebooks"] = w.codebooks
        sd[f"{name}.row_scales"] = w.row_scales
        if biases.get(name) is not None:
            sd[f"{name}.bias"] = biases[name]
        specs[name] = _linear_spec(w, biases.get(name) is not None, source_dtype)
    for name, t in (extra_tensors or {}).items():
        sd[name] = t
    sd = {k: v.detach().cpu().contiguous().clone() for k, v in sd.items()}
    shards: List[Dict[str, object]] = []
    cur: Dict[str, object] = {}
    cur_bytes = 0
    for name, t in sd.items():
        nb = t.numel() * t.element_size()
        if cur and cur_bytes + nb > max_shard_bytes:
            shards.append(cur)
            cur, cur_bytes = {name: t}, nb
        else:
            cur[name] = t
            cur_bytes += nb
    if cur or not shards:
        shards.append(cur)
    entries, records = [], {}
    for i, tensors in enumerate(shards):
        fname = f"shard-{i + 1:05d}-of-{len(shards):05d}.safetensors"
        path = out / fname
        safetensors.torch.save_file(tensors, str(path))
        entries.append(OQPackShardEntry(fname, _sha256(path), path.stat().st_size,
                                        tuple(tensors.keys())))
        for tname, t in tensors.items():
            layer = tname.rsplit(".", 1)[0]
            records[tname] = OQPackTensorRecord(tname, fname, _dtype_name(t), tuple(t.shape),
                                                t.numel() * t.element_size(),
                                                roles.get(tname, roles.get(layer, "other")))
    tok_files: List[str] = []
    if tokenizer_dir is not None and Path(tokenizer_dir).is_dir():
        for kf in _TOKENIZER_FILES:
            src = Path(tokenizer_dir) / kf
            if src.is_file():
                shutil.copy2(src, out / kf)
                tok_files.append(kf)
    if chat_template is not None:
        (out / "chat_template.jinja").write_text(chat_template, encoding="utf-8")
        if "chat_template.jinja" not in tok_files:
            tok_files.append("chat_template.jinja")
    elif (out / "chat_template.jinja").is_file():
        chat_template = (out / "chat_template.jinja").read_text(encoding="utf-8")
    manifest = OQPackManifest(OQPACK_FORMAT_VERSION, CODEC_SCHEMA_VERSION, str(model_id),
                              str(source_checkpoint_sha256), {}, {}, {}, None, entries, records,
                              specs, tok_files, chat_template)
    tmp = out / (MANIFEST_FILENAME + ".tmp")
    tmp.write_text(json.dumps(manifest.to_dict(), indent=2) + "\n", encoding="utf-8")
    tmp.replace(out / MANIFEST_FILENAME)
    return manifest


class LUTLayer:
    """One residual-VQ linear of a package on the GPU: ``weight`` is a
    math_engine.QuantizedWeight, ``bias`` fp32 or None; ``forward`` runs the
    multi-stage subspace LUT GEMM; ``native_linear`` repacks a single-stage
    8-bit block-16 layer into the tiled LUT-GEMV handle."""

    def __init__(self, name: str, weight, bias):
        self.name = name
        self.weight = weight
        self.bias = bias

    def forward(self, x):
        from .math_engine import subspace_lut_rvq_gemm
        return subspace_lut_rvq_gemm(x, self.weight, self.bias)

    __call__ = forward

    def native_linear(self):
        from .native import NativeSplitManifoldLinear
        w = self.weight
        if w.stages != 1 or w.bits_per_stage != 8 or w.block_size != 16:
            raise ValueError(f"{self.name}: the LUT-GEMV handle takes one 8-bit stage of block 16 "
                             f"(got {w.stages} x {w.bits_per_stage} bits, block {w.block_size})")
        rows, cols = w.original_shape
        if cols % 16:
            raise ValueError(f"{self.name}: in_features {cols} is not a multiple of 16")
        codes = w.packed_codes[0].reshape(rows, cols // 16).cpu().numpy()
        lin = NativeSplitManifoldLinear(cols, rows, 16, 256)
        bias = None if self.bias is None else self.bias.float().cpu().numpy()
        lin.initialize_weights(w.codebooks[0].cpu().numpy(), codes,
                               w.row_scales.float().cpu().numpy(), bias)
        return lin


def load_lut_layers(package_dir: Union[str, Path], *, device="cuda",
                    verify_checksums: bool = True, strict: bool = False):
    """Verify a package and return ({layer: LUTLayer}, manifest) for its
    adaptive_residual_vq linear / conv1d layers, tensors on `device`.  Layers
    of other codecs (Leech24, fused expert banks) are not on the LUT path:
    skipped, or an OQPackValidationError when strict."""
    import torch
    from .math_engine import QuantizedWeight
    pkg = Path(package_dir)
    manifest = verify_oqpack_integrity(pkg, verify_checksums=verify_checksums)
    tensors = open_oqpack_mmap(pkg, device="cpu", verify_checksums=False)
    layers: Dict[str, LUTLayer] = {}
    for name, spec in manifest.layer_specs.items():
        mtype = spec.get("module_type") or spec.get("type")
        codec = str(spec.get("codec", "adaptive_residual_vq"))
        if mtype not in ("linear", "residual_vq_linear", "conv1d", "residual_vq_conv1d") or \
                codec != "adaptive_residual_vq":
            if strict:
                raise OQPackValidationError(f"Layer {name}: {mtype} / {codec} is not a LUT layer")
            continue
        prefix = f"{name}." if name else ""
        try:
            packed = tensors[prefix + "packed_codes"]
            books = tensors[prefix + "codebooks"]
            scales = tensors[prefix + "row_scales"]
        except KeyError as e:
            raise OQPackValidationError(f"Missing tensors for layer {name}: {e}") from e
        w = QuantizedWeight(
            original_shape=(int(spec["out_features"]), int(spec["in_features"])),
            block_size=int(spec["block_size"]), bits_per_stage=int(spec["bits_per_stage"]),
            packed_codes=packed.to(device), codebooks=books.to(device=device, dtype=torch.float32),
            row_scales=scales.to(device=device, dtype=torch.float32), metrics={})
        if w.stages != int(spec["stages"]):
            raise OQPackValidationError(f"Layer {name}: {w.stages} stages stored, "
                                        f"{spec['stages']} declared")
        bias = tensors.get(prefix + "bias")
        has_bias = bool(spec.get("has_bias", spec.get("bias", False)))
        if has_bias and bias is None:
            raise OQPackValidationError(f"Missing tensors for layer {name}: bias")
        layers[name] = LUTLayer(name, w, None if bias is None else
                                bias.to(device=device, dtype=torch.float32))
    return layers, manifest
