"""GGUF checkpoints: an mmap reader, a writer, the Q4_K_M export and a Qwen3 loader.

Mirrors the reference's checkpoint and export surface:
  * ``open_gguf_mmap`` / ``GGUFMmap`` / ``GGUFTensorEntry`` -- src/torch2vk/checkpoints/gguf.py:100-303
    (header, metadata and tensor-info parsing, tensor views and row slices of the mapped file);
  * ``Q4KMQuantizationConfig``, ``export_q4_k_m_gguf`` -- src/torch2vk/quantize/gguf.py:33-139,191-247,363-429
    (per-tensor type policy, quantization of a safetensors checkpoint, GGUF v3 writer);
  * ``qwen3_q4_k_m_config`` -- src/models/quantized_qwen3/quantization.py:17-32.
The file format is the public GGUF v3 layout (little endian): magic "GGUF", version, tensor count,
metadata count, metadata key/values, tensor infos (name, dims innermost first, type, offset), padding
to the alignment, then the tensor data, each tensor at an aligned offset.

A quantized tensor's bytes are GGUF blocks row after row, which is exactly what the libt2h kernels
read, so loading is a copy of each tensor's bytes to the device.  Quantization for export runs on the
GPU quantizers (bit-identical to the reference's quantizers as restated in the CPU oracle).
"""

from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass
from enum import IntEnum
from pathlib import Path
from typing import BinaryIO, Iterable, Iterator

import numpy as np

GGUF_MAGIC = 0x46554747  # "GGUF" little endian
GGUF_VERSION = 3
GGUF_DEFAULT_ALIGNMENT = 32
GGUF_TYPE_MODEL = "model"
GGUF_FILE_TYPE_MOSTLY_Q4_K_M = 15
GGUF_QUANTIZATION_VERSION = 2


class GGUFTensorType(IntEnum):
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    I8 = 24
    I16 = 25
    I32 = 26
    I64 = 27
    F64 = 28
    BF16 = 30


class GGUFValueType(IntEnum):
    UINT8 = 0
    INT8 = 1
    UINT16 = 2
    INT16 = 3
    UINT32 = 4
    INT32 = 5
    FLOAT32 = 6
    BOOL = 7
    STRING = 8
    ARRAY = 9
    UINT64 = 10
    INT64 = 11
    FLOAT64 = 12


# (values per block, bytes per block) of the tensor types this build reads and writes
_BLOCK: dict[GGUFTensorType, tuple[int, int]] = {
    GGUFTensorType.F32: (1, 4),
    GGUFTensorType.F16: (1, 2),
    GGUFTensorType.BF16: (1, 2),
    GGUFTensorType.F64: (1, 8),
    GGUFTensorType.I8: (1, 1),
    GGUFTensorType.I16: (1, 2),
    GGUFTensorType.I32: (1, 4),
    GGUFTensorType.I64: (1, 8),
    GGUFTensorType.Q8_0: (32, 34),
    GGUFTensorType.Q2_K: (256, 84),
    GGUFTensorType.Q3_K: (256, 110),
    GGUFTensorType.Q4_K: (256, 144),
    GGUFTensorType.Q5_K: (256, 176),
    GGUFTensorType.Q6_K: (256, 210),
    GGUFTensorType.Q8_K: (256, 292),
}

# scalar metadata encodings: struct format per value type
_SCALAR_FMT = {
    GGUFValueType.UINT8: "<B", GGUFValueType.INT8: "<b", GGUFValueType.UINT16: "<H", GGUFValueType.INT16: "<h",
    GGUFValueType.UINT32: "<I", GGUFValueType.INT32: "<i", GGUFValueType.FLOAT32: "<f",
    GGUFValueType.UINT64: "<Q", GGUFValueType.INT64: "<q", GGUFValueType.FLOAT64: "<d",
}

# libt2h type names of the GGUF types the kernels consume
KERNEL_TYPE = {GGUFTensorType.Q4_K: "q4_k", GGUFTensorType.Q6_K: "q6_k", GGUFTensorType.Q8_0: "q8_0"}


def tensor_nbytes(ggml_type: GGUFTensorType, logical_shape: tuple[int, ...]) -> int:
    """Bytes of a tensor; the innermost dimension must be a whole number of blocks."""
    try:
        block, size = _BLOCK[GGUFTensorType(ggml_type)]
    except KeyError as exc:
        raise ValueError(f"unsupported GGUF tensor type {GGUFTensorType(ggml_type).name}") from exc
    if not logical_shape:
        return size
    if logical_shape[-1] % block:
        raise ValueError(f"{GGUFTensorType(ggml_type).name} row of {logical_shape[-1]} values is not a whole "
                         f"number of {block}-value blocks")
    n = 1
    for d in logical_shape:
        n *= int(d)
    return n // block * size


# ------------------------------------------------------------------------------------------- reader


@dataclass(frozen=True)
class GGUFTensorEntry:
    """One tensor of a GGUF file.  ``logical_shape`` is outermost first (rows, values per row);
    ``ggml_shape`` is the file's order, innermost first."""
    name: str
    ggml_type: GGUFTensorType
    ggml_shape: tuple[int, ...]
    logical_shape: tuple[int, ...]
    data_offset: int  # absolute byte offset in the file
    nbytes: int

    @property
    def row_bytes(self) -> int:
        rows = self.logical_shape[0] if len(self.logical_shape) > 1 else 1
        return self.nbytes // rows


class _Reader:
    def __init__(self, handle: BinaryIO) -> None:
        self.h = handle

    def raw(self, n: int) -> bytes:
        b = self.h.read(n)
        if len(b) != n:
            raise ValueError("truncated GGUF file")
        return b

    def scalar(self, fmt: str):
        return struct.unpack(fmt, self.raw(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        return self.raw(self.scalar("<Q")).decode("utf-8")

    def value(self, vtype: GGUFValueType):
        if vtype in _SCALAR_FMT:
            return self.scalar(_SCALAR_FMT[vtype])
        if vtype is GGUFValueType.BOOL:
            return bool(self.scalar("<B"))
        if vtype is GGUFValueType.STRING:
            return self.string()
        if vtype is GGUFValueType.ARRAY:
            etype = GGUFValueType(self.scalar("<I"))
            count = self.scalar("<Q")
            return [self.value(etype) for _ in range(count)]
        raise ValueError(f"unsupported GGUF metadata type {vtype}")


def _alignment(metadata: dict[str, object]) -> int:
    a = metadata.get("general.alignment", GGUF_DEFAULT_ALIGNMENT)
    if not isinstance(a, int) or a <= 0 or a & (a - 1):
        raise ValueError(f"GGUF general.alignment must be a power of two, got {a!r}")
    return a


def read_gguf_index(path: str | Path) -> tuple[dict[str, GGUFTensorEntry], dict[str, object]]:
    """Parse the header, metadata and tensor infos (no tensor data is read)."""
    path = Path(path)
    with path.open("rb") as f:
        r = _Reader(f)
        magic = r.scalar("<I")
        if magic != GGUF_MAGIC:
            raise ValueError(f"{path} is not a GGUF file (magic 0x{magic:08x})")
        version = r.scalar("<I")
        if version not in (2, 3):
            raise ValueError(f"unsupported GGUF version {version} in {path}")
        n_tensors = r.scalar("<Q")
        n_kv = r.scalar("<Q")
        metadata: dict[str, object] = {"GGUF.version": version}
        for _ in range(n_kv):
            key = r.string()
            metadata[key] = r.value(GGUFValueType(r.scalar("<I")))
        infos = []
        for _ in range(n_tensors):
            name = r.string()
            dims = tuple(r.scalar("<Q") for _ in range(r.scalar("<I")))
            ggml_type = GGUFTensorType(r.scalar("<I"))
            infos.append((name, dims, ggml_type, r.scalar("<Q")))
        align = _alignment(metadata)
        data_start = -(-f.tell() // align) * align
    tensors = {}
    for name, dims, ggml_type, offset in infos:
        if name in tensors:
            raise ValueError(f"duplicate GGUF tensor {name!r}")
        logical = tuple(reversed(dims))
        tensors[name] = GGUFTensorEntry(name=name, ggml_type=ggml_type, ggml_shape=dims, logical_shape=logical,
                                        data_offset=data_start + offset, nbytes=tensor_nbytes(ggml_type, logical))
    return tensors, metadata


class GGUFMmap:
    """A GGUF file mapped read-only: metadata, tensor entries, zero-copy tensor views and row slices."""

    def __init__(self, path: str | Path) -> None:
        self.path = Path(path)
        self.tensors, self.metadata = read_gguf_index(self.path)
        self._file = None
        self._map = None

    def __enter__(self) -> "GGUFMmap":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def close(self) -> None:
        """Release the mapping; arrays still viewing it keep it alive until they are dropped."""
        if self._map is not None:
            try:
                self._map.close()
            except BufferError:
                pass  # views handed out by array()/buffer_slice() are still referenced
            self._map = None
        if self._file is not None:
            self._file.close()
            self._file = None

    def entry(self, name: str) -> GGUFTensorEntry:
        try:
            return self.tensors[name]
        except KeyError as exc:
            raise KeyError(f"no GGUF tensor {name!r}; the file has {len(self.tensors)} tensors") from exc

    def _mapped(self) -> mmap.mmap:
        if self._map is None:
            self._file = self.path.open("rb")
            self._map = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ)
        return self._map

    def buffer_slice(self, name: str) -> memoryview:
        e = self.entry(name)
        m = self._mapped()
        if e.data_offset + e.nbytes > len(m):
            raise ValueError(f"GGUF tensor {name!r} runs past the end of {self.path}")
        return memoryview(m)[e.data_offset:e.data_offset + e.nbytes]

    def buffer_rows(self, name: str, *, row_offset: int, row_count: int) -> memoryview:
        e = self.entry(name)
        rows = e.logical_shape[0] if len(e.logical_shape) > 1 else 1
        if row_offset < 0 or row_count <= 0 or row_offset + row_count > rows:
            raise ValueError(f"rows [{row_offset}, {row_offset + row_count}) outside {name!r} with {rows} rows")
        return self.buffer_slice(name)[row_offset * e.row_bytes:(row_offset + row_count) * e.row_bytes]

    def array(self, name: str) -> np.ndarray:
        """The tensor's bytes as a read-only uint8 array [rows, row bytes] (a view of the mapping)."""
        e = self.entry(name)
        a = np.frombuffer(self.buffer_slice(name), dtype=np.uint8)
        return a.reshape(e.logical_shape[0], e.row_bytes) if len(e.logical_shape) > 1 else a

    def float_array(self, name: str) -> np.ndarray:
        """An F32 / F16 / BF16 tensor as a float32 copy, logical shape."""
        e = self.entry(name)
        raw = np.frombuffer(self.buffer_slice(name), dtype=np.uint8)
        if e.ggml_type is GGUFTensorType.F32:
            out = raw.view(np.float32)
        elif e.ggml_type is GGUFTensorType.F16:
            out = raw.view(np.float16).astype(np.float32)
        elif e.ggml_type is GGUFTensorType.BF16:
            out = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        else:
            raise TypeError(f"GGUF tensor {name!r} is {e.ggml_type.name}, not a float type")
        return np.array(out.reshape(e.logical_shape), dtype=np.float32, copy=True)


def open_gguf_mmap(path: str | Path) -> GGUFMmap:
    return GGUFMmap(path)


# ------------------------------------------------------------------------------------------- writer


@dataclass(frozen=True)
class GGUFTensor:
    """A tensor to write: ``data`` holds its bytes in file order (quantized blocks row after row)."""
    name: str
    ggml_type: GGUFTensorType
    logical_shape: tuple[int, ...]
    data: np.ndarray

    def __post_init__(self) -> None:
        want = tensor_nbytes(self.ggml_type, self.logical_shape)
        if np.asarray(self.data).nbytes != want:
            raise ValueError(f"tensor {self.name!r}: {np.asarray(self.data).nbytes} bytes, "
                             f"{GGUFTensorType(self.ggml_type).name}{self.logical_shape} needs {want}")


@dataclass(frozen=True)
class GGUFMetadataValue:
    key: str
    value_type: GGUFValueType
    value: object
    element_type: GGUFValueType | None = None  # ARRAY only


def _infer_value(key: str, value) -> GGUFMetadataValue:
    if isinstance(value, GGUFMetadataValue):
        return value
    if isinstance(value, bool):
        return GGUFMetadataValue(key, GGUFValueType.BOOL, value)
    if isinstance(value, int):
        return GGUFMetadataValue(key, GGUFValueType.UINT32 if 0 <= value < 2**32 else GGUFValueType.INT64, value)
    if isinstance(value, float):
        return GGUFMetadataValue(key, GGUFValueType.FLOAT32, value)
    if isinstance(value, str):
        return GGUFMetadataValue(key, GGUFValueType.STRING, value)
    if isinstance(value, (list, tuple)):
        if not value:
            raise ValueError(f"metadata {key!r}: an empty array needs an explicit element type")
        return GGUFMetadataValue(key, GGUFValueType.ARRAY, list(value), _infer_value(key, value[0]).value_type)
    raise TypeError(f"metadata {key!r}: unsupported value {value!r}")


class _Writer:
    def __init__(self, handle: BinaryIO) -> None:
        self.h = handle

    def scalar(self, fmt: str, v) -> None:
        self.h.write(struct.pack(fmt, v))

    def string(self, s: str) -> None:
        b = s.encode("utf-8")
        self.scalar("<Q", len(b))
        self.h.write(b)

    def value(self, vtype: GGUFValueType, v, etype: GGUFValueType | None = None) -> None:
        if vtype in _SCALAR_FMT:
            self.scalar(_SCALAR_FMT[vtype], v)
        elif vtype is GGUFValueType.BOOL:
            self.scalar("<B", 1 if v else 0)
        elif vtype is GGUFValueType.STRING:
            self.string(v)
        elif vtype is GGUFValueType.ARRAY:
            if etype is None or etype is GGUFValueType.ARRAY:
                raise ValueError("GGUF arrays need a scalar or string element type")
            self.scalar("<I", int(etype))
            self.scalar("<Q", len(v))
            for x in v:
                self.value(etype, x)
        else:
            raise ValueError(f"unsupported GGUF metadata type {vtype}")


def write_gguf(path: str | Path, metadata: dict[str, object] | Iterable[GGUFMetadataValue],
               tensors: Iterable[GGUFTensor]) -> Path:
    """Write a GGUF v3 file.  Metadata values may be given as python values (uint32 for non-negative
    ints, float32, bool, string, arrays thereof) or as ``GGUFMetadataValue`` for an explicit type."""
    path = Path(path)
    items = ([_infer_value(k, v) for k, v in metadata.items()] if isinstance(metadata, dict)
             else [_infer_value(m.key, m) for m in metadata])
    align = _alignment({m.key: m.value for m in items})
    tensors = list(tensors)
    offsets, cur = [], 0
    for t in tensors:
        offsets.append(cur)
        cur += -(-np.asarray(t.data).nbytes // align) * align
    with path.open("wb") as f:
        w = _Writer(f)
        w.scalar("<I", GGUF_MAGIC)
        w.scalar("<I", GGUF_VERSION)
        w.scalar("<Q", len(tensors))
        w.scalar("<Q", len(items))
        for m in items:
            w.string(m.key)
            w.scalar("<I", int(m.value_type))
            w.value(m.value_type, m.value, m.element_type)
        for t, off in zip(tensors, offsets):
            w.string(t.name)
            w.scalar("<I", len(t.logical_shape))
            for d in reversed(t.logical_shape):
                w.scalar("<Q", int(d))
            w.scalar("<I", int(t.ggml_type))
            w.scalar("<Q", off)
        f.write(bytes(-f.tell() % align))
        for t in tensors:
            b = np.ascontiguousarray(t.data).tobytes()
            f.write(b)
            f.write(bytes(-len(b) % align))
    return path


# ------------------------------------------------------------------------------- Q4_K_M export


@dataclass(frozen=True)
class Q4KMQuantizationConfig:
    """Per-tensor GGUF type policy of the reference's Q4_K_M export (src/torch2vk/quantize/gguf.py:33-83):
    tensors named in q6/q8 (or under their prefixes) are forced to Q6_K / Q8_0 when 2-D or more;
    otherwise a 2-D tensor is Q4_K when its rows are whole 256-value blocks, Q8_0 when whole 32-value
    blocks, else F32; other ranks and non-float32 checkpoints stay F32; f16 names stay F16."""
    model_name: str
    gguf_arch: str
    f16_tensor_names: tuple[str, ...] = ()
    f16_tensor_prefixes: tuple[str, ...] = ()
    q6_tensor_names: tuple[str, ...] = ()
    q6_tensor_prefixes: tuple[str, ...] = ()
    q8_tensor_names: tuple[str, ...] = ()
    q8_tensor_prefixes: tuple[str, ...] = ()
    extra_uint32_metadata: tuple[tuple[str, int], ...] = ()

    def gguf_type(self, *, checkpoint_key: str, shape: tuple[int, ...], dtype: str = "float32") -> GGUFTensorType:
        named = lambda names, prefixes: checkpoint_key in names or checkpoint_key.startswith(prefixes)  # noqa: E731
        if named(self.f16_tensor_names, self.f16_tensor_prefixes):
            return GGUFTensorType.F16
        if dtype not in ("float32", "float16", "bfloat16") and not dtype.startswith("float8"):
            return GGUFTensorType.F32
        if named(self.q8_tensor_names, self.q8_tensor_prefixes) and len(shape) >= 2:
            return GGUFTensorType.Q8_0
        if named(self.q6_tensor_names, self.q6_tensor_prefixes) and len(shape) >= 2:
            return GGUFTensorType.Q6_K
        if len(shape) != 2:
            return GGUFTensorType.F32
        if shape[-1] % 256 == 0:
            return GGUFTensorType.Q4_K
        if shape[-1] % 32 == 0:
            return GGUFTensorType.Q8_0
        return GGUFTensorType.F32

    def metadata(self) -> list[GGUFMetadataValue]:
        out = [
            GGUFMetadataValue("general.architecture", GGUFValueType.STRING, self.gguf_arch),
            GGUFMetadataValue("general.name", GGUFValueType.STRING, self.model_name),
            GGUFMetadataValue("general.type", GGUFValueType.STRING, GGUF_TYPE_MODEL),
            GGUFMetadataValue("general.file_type", GGUFValueType.UINT32, GGUF_FILE_TYPE_MOSTLY_Q4_K_M),
            GGUFMetadataValue("general.quantization_version", GGUFValueType.UINT32, GGUF_QUANTIZATION_VERSION),
        ]
        out += [GGUFMetadataValue(k, GGUFValueType.UINT32, v) for k, v in self.extra_uint32_metadata]
        return out


def qwen3_q4_k_m_config(num_hidden_layers: int) -> Q4KMQuantizationConfig:
    """Qwen3's Q4_K_M topology: Q6_K lm_head, and v_proj / down_proj on the more-bits layers."""
    from torch2vk_amd.qwen3.config import q4_k_m_more_bits_layer_indices

    more = q4_k_m_more_bits_layer_indices(num_hidden_layers)
    return Q4KMQuantizationConfig(
        model_name="Qwen3", gguf_arch="qwen3",
        q6_tensor_names=("lm_head.weight",
                         *(f"model.layers.{i}.self_attn.v_proj.weight" for i in more),
                         *(f"model.layers.{i}.mlp.down_proj.weight" for i in more)))


def _iter_safetensors(model_dir: Path) -> Iterator[tuple[str, "object"]]:
    from safetensors import safe_open

    paths = sorted(model_dir.glob("*.safetensors"))
    if not paths:
        raise FileNotFoundError(f"no *.safetensors in {model_dir}")
    for p in paths:
        with safe_open(p, framework="pt", device="cpu") as ck:
            for name in ck.keys():
                yield name, ck.get_tensor(name)


def quantize_tensor(name: str, tensor, config: Q4KMQuantizationConfig, device) -> GGUFTensor:
    """One checkpoint tensor in its GGUF type; quantized types go through the GPU quantizers."""
    import torch

    from torch2vk_amd import kernels

    shape = tuple(int(d) for d in tensor.shape)
    dtype = str(tensor.dtype).removeprefix("torch.")
    gtype = config.gguf_type(checkpoint_key=name, shape=shape, dtype=dtype)
    if gtype is GGUFTensorType.F16:
        return GGUFTensor(name, gtype, shape, tensor.to(torch.float16).cpu().numpy())
    if gtype is GGUFTensorType.F32:
        return GGUFTensor(name, gtype, shape, tensor.to(torch.float32).cpu().numpy())
    rows = shape[0]
    cols = 1
    for d in shape[1:]:
        cols *= d
    dense = tensor.to(device=device, dtype=torch.float32).reshape(rows, cols)
    if gtype is GGUFTensorType.Q8_0 and cols % 32:
        padded = torch.zeros(rows, -(-cols // 32) * 32, dtype=torch.float32, device=device)
        padded[:, :cols] = dense
        dense, cols = padded, padded.shape[1]
    packed = kernels.quantize(dense.contiguous(), KERNEL_TYPE[gtype])
    return GGUFTensor(name, gtype, (rows, cols), packed.cpu().numpy())


def export_q4_k_m_gguf(*, model_dir: str | Path, output: str | Path, config: Q4KMQuantizationConfig,
                       overwrite: bool = False, device=None) -> Path:
    """Quantize every tensor of a safetensors checkpoint per ``config`` on the GPU and write a GGUF v3
    file (src/torch2vk/quantize/gguf.py:191-247).  An existing file that already matches the policy is
    kept unless ``overwrite``."""
    import torch

    output = Path(output).expanduser().resolve()
    if output.exists() and not overwrite and _matches(output, config):
        return output
    device = torch.device(device) if device is not None else torch.device("cuda:0")
    tensors, seen = [], set()
    for name, t in _iter_safetensors(Path(model_dir).expanduser().resolve()):
        if name in seen:
            raise ValueError(f"duplicate checkpoint tensor {name!r}")
        seen.add(name)
        tensors.append(quantize_tensor(name, t, config, device))
    output.parent.mkdir(parents=True, exist_ok=True)
    tmp = output.with_name(output.name + ".tmp")
    write_gguf(tmp, config.metadata(), tensors)
    tmp.replace(output)
    return output


def _matches(path: Path, config: Q4KMQuantizationConfig) -> bool:
    try:
        tensors, metadata = read_gguf_index(path)
    except (OSError, ValueError):
        return False
    if metadata.get("general.file_type") != GGUF_FILE_TYPE_MOSTLY_Q4_K_M:
        return False
    if any(metadata.get(k) != v for k, v in config.extra_uint32_metadata):
        return False
    return all(e.ggml_type is config.gguf_type(checkpoint_key=n, shape=e.logical_shape) for n, e in tensors.items())


# ------------------------------------------------------------------------------------ Qwen3 loader

# checkpoint name -> decoder name (HF Qwen3ForCausalLM parameter names, as the reference exports them)
def qwen3_tensor_names(layers: int) -> dict[str, str]:
    names = {"model.embed_tokens.weight": "embed", "lm_head.weight": "lm_head", "model.norm.weight": "norm"}
    for i in range(layers):
        p, q = f"model.layers.{i}.", f"layers.{i}."
        for proj in ("q", "k", "v", "o"):
            names[f"{p}self_attn.{proj}_proj.weight"] = q + proj
        for proj in ("gate", "up", "down"):
            names[f"{p}mlp.{proj}_proj.weight"] = q + proj
        names[p + "input_layernorm.weight"] = q + "input_norm"
        names[p + "post_attention_layernorm.weight"] = q + "post_norm"
        names[p + "self_attn.q_norm.weight"] = q + "q_norm"
        names[p + "self_attn.k_norm.weight"] = q + "k_norm"
    return names


def load_qwen3_gguf(path: str | Path, config, *, device) -> "object":
    """A Qwen3 GGUF file (HF tensor names) as decoder weights on ``device``: quantized tensors are copied
    byte for byte (their rows are the kernels' layout), norm weights as fp32.  A checkpoint with tied
    embeddings (no lm_head.weight) uses the embedding rows for the LM head."""
    import torch

    from torch2vk_amd.qwen3.weights import Qwen3Weights, matrix_shapes, norm_shapes, stack_qkv

    names = qwen3_tensor_names(config.layers)
    mats, norms = matrix_shapes(config), norm_shapes(config)
    w = Qwen3Weights(config=config, policy="gguf")
    with open_gguf_mmap(path) as g:
        present = {names[n]: n for n in g.tensors if n in names}
        if "lm_head" not in present and "embed" in present:
            present["lm_head"] = present["embed"]
        for key, (rows, cols) in mats.items():
            if key not in present:
                raise KeyError(f"{path}: no tensor for {key} ({[k for k, v in names.items() if v == key][0]})")
            e = g.entry(present[key])
            if e.ggml_type not in KERNEL_TYPE:
                raise TypeError(f"{e.name}: {e.ggml_type.name} is not a type the decode kernels read")
            if e.logical_shape != (rows, cols):
                raise ValueError(f"{e.name}: shape {e.logical_shape}, the config needs {(rows, cols)}")
            w.packed[key] = torch.from_numpy(g.array(e.name).copy()).to(device)
            w.types[key] = KERNEL_TYPE[e.ggml_type]
        for key, n in norms.items():
            if key not in present:
                raise KeyError(f"{path}: no tensor for {key}")
            v = g.float_array(present[key])
            if v.shape != (n,):
                raise ValueError(f"{present[key]}: shape {v.shape}, the config needs ({n},)")
            w.norms[key] = torch.from_numpy(v.copy()).to(device)
    stack_qkv(w)
    return w
