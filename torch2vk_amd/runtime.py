"""The reference's operator-call surface over libt2h: shader variants called as ``VARIANT(rt, **tensors)``.

In torch2vk every kernel is a ``ShaderVariant`` whose ``ShaderContract`` lists its tensor fields (name, io kind,
dtype, symbolic shape, layout) and its dynamic scalars; calling the variant forwards to ``rt.dispatch``, which
checks the arguments against the contract, binds the shape symbols and launches
(src/torch2vk/runtime/shader.py:77-200, src/torch2vk/runtime/dispatcher.py:28-109).  Here the same objects
carry a ``launch`` callable instead of GLSL: once ``RuntimeSession.dispatch`` has checked the call, the launch
runs one ``t2h_*`` entry point (through ``torch2vk_amd.kernels``) on the session's stream.  The checks raise
the reference's exceptions before anything is launched: ValueError for missing, extra or mis-shaped fields and
unresolved symbols, TypeError for a field that is not a tensor or has the wrong dtype.

Tensors are torch tensors on the session's device.  Quantized weights use the reference's physical types:
Q4_K as uint32 words [N, ceil(K/256)*36], Q6_K as uint16 halfwords [N, ceil(K/256)*105], Q8_0 as uint16
halfwords [N, ceil(K/32)*17] (src/torch2vk/vulkan/types.py:64-82); the launches view them as the bytes the
kernels read, without a copy.  Activations are bf16 and the residual stream fp32, where the reference uses fp16.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum
from typing import Callable, Mapping, Union

import torch


class IOKind(str, Enum):
    INPUT = "input"
    OUTPUT = "output"
    INOUT = "inout"


# ------------------------------------------------------------ shape expressions --

@dataclass(frozen=True)
class CeilDivExpr:
    lhs: "ExprDim"
    rhs: "ExprDim"


@dataclass(frozen=True)
class MulExpr:
    lhs: "ExprDim"
    rhs: "ExprDim"


@dataclass(frozen=True)
class AddExpr:
    lhs: "ExprDim"
    rhs: "ExprDim"


ExprDim = Union[int, str, CeilDivExpr, MulExpr, AddExpr]


def ceil_div(lhs: ExprDim, rhs: ExprDim) -> CeilDivExpr:
    return CeilDivExpr(lhs, rhs)


def mul(lhs: ExprDim, rhs: ExprDim) -> MulExpr:
    return MulExpr(lhs, rhs)


def add(lhs: ExprDim, rhs: ExprDim) -> AddExpr:
    return AddExpr(lhs, rhs)


def eval_expr(expr: ExprDim, symbols: Mapping[str, int]) -> int:
    """Value of a shape expression under bound symbols (src/torch2vk/runtime/shader.py:250-268)."""
    if isinstance(expr, int):
        return int(expr)
    if isinstance(expr, str):
        if expr not in symbols:
            raise ValueError(f"Unresolved shape symbol {expr!r}")
        return int(symbols[expr])
    if isinstance(expr, CeilDivExpr):
        lhs, rhs = eval_expr(expr.lhs, symbols), eval_expr(expr.rhs, symbols)
        if rhs <= 0:
            raise ValueError(f"ceil_div rhs must be positive, got {rhs}")
        return (lhs + rhs - 1) // rhs
    if isinstance(expr, MulExpr):
        return eval_expr(expr.lhs, symbols) * eval_expr(expr.rhs, symbols)
    if isinstance(expr, AddExpr):
        return eval_expr(expr.lhs, symbols) + eval_expr(expr.rhs, symbols)
    raise TypeError(f"Unsupported expression dim {expr!r}")


# ------------------------------------------------------------------ contracts --

CONTIGUOUS = "contiguous"
Q4_K_WORDS = "q4_k_words"          # uint32 [N, ceil(K/256)*36]
Q6_K_HALFWORDS = "q6_k_halfwords"  # uint16 [N, ceil(K/256)*105]
Q8_0_HALFWORDS = "q8_0_halfwords"  # uint16 [N, ceil(K/32)*17]

_DTYPES = {
    "bfloat16": torch.bfloat16, "float32": torch.float32, "float16": torch.float16, "uint32": torch.uint32,
    "uint16": torch.uint16, "uint8": torch.uint8, "int32": torch.int32, "int64": torch.int64,
}


@dataclass(frozen=True)
class TensorContract:
    dtype: str | tuple[str, ...]
    shape: tuple[ExprDim, ...]
    layout: str = CONTIGUOUS

    def dtypes(self) -> tuple[torch.dtype, ...]:
        names = (self.dtype,) if isinstance(self.dtype, str) else self.dtype
        return tuple(_DTYPES[n] for n in names)


@dataclass(frozen=True)
class TensorFieldSpec:
    name: str
    io_kind: IOKind
    role: str
    contract: TensorContract


@dataclass(frozen=True)
class PushConstantInput:
    """A dynamic scalar passed by name at the call (the reference's PushConstantInput, shader.py:94-99).  An
    unsigned input (``kind`` "uint32", the default) is a Python int or a one-element int32 device tensor, so a
    captured graph can replay it with new values; a "float32" input (ROPE_TABLE_F32's theta) is a Python
    number."""
    name: str
    kind: str = "uint32"

    def __post_init__(self) -> None:
        if self.kind not in ("uint32", "float32"):
            raise ValueError(f"push input {self.name!r}: kind must be uint32 or float32, got {self.kind!r}")


@dataclass(frozen=True)
class ShaderContract:
    class_name: str
    shader_name: str
    fields: tuple[TensorFieldSpec, ...]
    push_inputs: tuple[PushConstantInput, ...] = ()

    @property
    def input_fields(self) -> tuple[TensorFieldSpec, ...]:
        return tuple(f for f in self.fields if f.io_kind in (IOKind.INPUT, IOKind.INOUT))

    @property
    def output_fields(self) -> tuple[TensorFieldSpec, ...]:
        return tuple(f for f in self.fields if f.io_kind in (IOKind.OUTPUT, IOKind.INOUT))

    def validate_definition(self) -> None:
        if not self.class_name or not self.shader_name:
            raise ValueError("ShaderContract needs a class_name and a shader_name")
        names = [f.name for f in self.fields] + [p.name for p in self.push_inputs]
        if len(set(names)) != len(names):
            raise ValueError(f"{self.shader_name} has duplicate field names")


Launch = Callable[["RuntimeSession", Mapping[str, torch.Tensor], Mapping[str, int], Mapping[str, object]], None]


@dataclass(frozen=True)
class ShaderVariant:
    """A kernel entry point with its contract; ``VARIANT(rt, **tensors)`` dispatches it on ``rt``."""
    name: str
    family: str
    contract: ShaderContract
    launch: Launch = field(compare=False, repr=False)

    def __post_init__(self) -> None:
        if self.name != self.contract.shader_name:
            raise ValueError(f"ShaderVariant name {self.name!r} must equal contract shader_name")
        self.contract.validate_definition()

    def __call__(self, rt: "RuntimeSession", **arguments: object) -> None:
        rt.dispatch(self, **arguments)


# -------------------------------------------------------------------- session --

@dataclass(frozen=True)
class DispatchRecord:
    index: int
    shader: str
    symbols: tuple[tuple[str, int], ...]


class RuntimeSession:
    """Owns the device, the caller-visible dispatch log and the kernels' scratch workspaces (allocated once per
    size, reused by every later dispatch); ``dispatch`` checks a call against its contract and launches it."""

    def __init__(self, device: torch.device | str = "cuda:0", *, record: bool = False) -> None:
        self.device = torch.device(device)
        self.record = record
        self.records: list[DispatchRecord] = []
        self._workspaces: dict[tuple[str, int], torch.Tensor] = {}

    def workspace(self, key: str, nbytes: int) -> torch.Tensor:
        """A uint8 device buffer of at least nbytes, kept for later dispatches under ``key``."""
        t = self._workspaces.get((key, nbytes))
        if t is None:
            t = torch.zeros(nbytes, dtype=torch.uint8, device=self.device)
            self._workspaces[(key, nbytes)] = t
        return t

    def dispatch(self, variant: ShaderVariant, **arguments: object) -> None:
        contract = variant.contract
        expected = {f.name for f in contract.fields}
        push_names = {p.name for p in contract.push_inputs}
        provided = set(arguments)
        if missing := expected - provided:
            raise ValueError(f"{variant.name} missing tensor fields: {sorted(missing)}")
        if missing_push := push_names - provided:
            raise ValueError(f"{variant.name} missing push constant inputs: {sorted(missing_push)}")
        if extra := provided - expected - push_names:
            raise ValueError(f"{variant.name} got unexpected fields: {sorted(extra)}")
        tensors: dict[str, torch.Tensor] = {}
        for f in contract.fields:
            t = arguments[f.name]
            if not isinstance(t, torch.Tensor):
                raise TypeError(f"{variant.name}.{f.name} expects a tensor, got {type(t).__name__}")
            if t.device != self.device:
                raise ValueError(f"{variant.name}.{f.name} is on {t.device}, the session runs on {self.device}")
            if t.dtype not in f.contract.dtypes():
                raise TypeError(f"{variant.name}.{f.name} dtype {t.dtype} not in {f.contract.dtype}")
            if not t.is_contiguous():
                raise ValueError(f"{variant.name}.{f.name} must be contiguous ({f.contract.layout} layout)")
            if t.dim() != len(f.contract.shape):
                raise ValueError(f"{variant.name}.{f.name} rank {t.dim()} != contract rank {len(f.contract.shape)}")
            tensors[f.name] = t
        symbols = self._bind_shape_symbols(variant, tensors)
        push: dict[str, object] = {}
        for p in contract.push_inputs:
            v = arguments[p.name]
            if p.kind == "float32":
                if isinstance(v, bool) or not isinstance(v, (int, float)):
                    raise TypeError(f"{variant.name}.{p.name} must be a number, got {type(v).__name__}")
                push[p.name] = float(v)
                continue
            if isinstance(v, torch.Tensor):
                if v.dtype != torch.int32 or v.numel() != 1 or v.device != self.device:
                    raise TypeError(f"{variant.name}.{p.name} must be an int or a one-element int32 device tensor")
            elif not isinstance(v, int) or isinstance(v, bool) or v < 0:
                raise TypeError(f"{variant.name}.{p.name} must be a non-negative int or an int32 device tensor")
            push[p.name] = v
        if self.record:
            self.records.append(DispatchRecord(len(self.records), variant.name, tuple(sorted(symbols.items()))))
        variant.launch(self, tensors, symbols, push)

    @staticmethod
    def _bind_shape_symbols(variant: ShaderVariant, tensors: Mapping[str, torch.Tensor]) -> dict[str, int]:
        """Bind every bare symbol to the size it meets first, then require every dimension (bare symbols met
        again, literals and expressions over symbols) to equal what the contract says."""
        symbols: dict[str, int] = {}
        for f in variant.contract.fields:
            for axis, dim in enumerate(f.contract.shape):
                if isinstance(dim, str) and dim not in symbols:
                    symbols[dim] = int(tensors[f.name].shape[axis])
        for f in variant.contract.fields:
            for axis, dim in enumerate(f.contract.shape):
                want = eval_expr(dim, symbols)
                got = int(tensors[f.name].shape[axis])
                if got != want:
                    raise ValueError(f"{variant.name}.{f.name} axis {axis}: size {got}, contract {dim!r} = {want}")
        return symbols


# ------------------------------------------------------- quantized-linear choice --

def weight_layout(weight: torch.Tensor, k: int) -> str:
    """The GGUF layout a weight tensor carries, from its physical dtype and row width for logical K:
    Q4_K words, Q6_K halfwords or Q8_0 halfwords (src/torch2vk/vulkan/types.py:64-82)."""
    if weight.dim() != 2:
        raise ValueError(f"weight must be rank 2, got shape {tuple(weight.shape)}")
    width = int(weight.shape[1])
    if weight.dtype == torch.uint32 and width == (k + 255) // 256 * 36:
        return Q4_K_WORDS
    if weight.dtype == torch.uint16 and width == (k + 255) // 256 * 105:
        return Q6_K_HALFWORDS
    if weight.dtype == torch.uint16 and width == (k + 31) // 32 * 17:
        return Q8_0_HALFWORDS
    raise ValueError(f"weight {tuple(weight.shape)} {weight.dtype}: expected Q4_K, Q6_K, or Q8_0 layout for K={k}")


def run_quantized_linear(rt: RuntimeSession, *, q4: ShaderVariant, q6: ShaderVariant, q8: ShaderVariant,
                         x: torch.Tensor, weight: torch.Tensor, output: torch.Tensor) -> None:
    """Run the variant of the weight's layout (src/torch2vk/runtime/quantized_dispatch.py:15-35)."""
    layout = weight_layout(weight, int(x.shape[-1]))
    variant = {Q4_K_WORDS: q4, Q6_K_HALFWORDS: q6, Q8_0_HALFWORDS: q8}[layout]
    variant(rt, x=x, weight=weight, output=output)
