"""CPU oracle for torch2vk's GGUF block formats (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker.  The shipped path
(``torch2vk_amd``) never imports it.

Two kinds of functions live here:

* ``quantize_*`` / ``dequant_*`` call the C restatement in ``q_oracle.c`` of the
  reference GLSL quantizers (``/root/reference/src/torch2vk/quantize/vulkan.py``).
* ``decode_q4_k_*`` / ``decode_q6_k_codes`` / ``decode_q8_0_codes`` restate, in
  numpy, the *decoders* the reference's kernels use.  They read the packed
  bytes with the reference kernels' own bit arithmetic, independently of the
  C packer, so agreement between them and the packer pins the byte layout.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "liboracle.so"
_lib: ctypes.CDLL | None = None

Q4_K_BLOCK_BYTES = 144
Q6_K_BLOCK_BYTES = 210
Q8_0_BLOCK_BYTES = 34


def build(force: bool = False) -> Path:
    """Compile ``q_oracle.c`` with the committed Makefile (gcc, no fp contraction)."""
    if force or not _LIB_PATH.exists() or _LIB_PATH.stat().st_mtime < (_HERE / "q_oracle.c").stat().st_mtime:
        subprocess.run(["make", "-B" if force else "-s", "_build/liboracle.so"], cwd=_HERE, check=True)
    return _LIB_PATH


def _load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        f32p = ctypes.POINTER(ctypes.c_float)
        u8p = ctypes.POINTER(ctypes.c_uint8)
        for name in ("oracle_quantize_q4_k", "oracle_quantize_q6_k", "oracle_quantize_q8_0"):
            fn = getattr(lib, name)
            fn.argtypes = [f32p, ctypes.c_int64, ctypes.c_int64, u8p]
            fn.restype = None
        for name in ("oracle_dequant_q4_k", "oracle_dequant_q6_k", "oracle_dequant_q8_0"):
            fn = getattr(lib, name)
            fn.argtypes = [u8p, ctypes.c_int64, ctypes.c_int64, f32p]
            fn.restype = None
        lib.oracle_q4_k_subblocks.argtypes = [f32p, ctypes.c_int64, f32p, f32p]
        lib.oracle_q4_k_subblocks.restype = None
        lib.oracle_q6_k_subblocks.argtypes = [f32p, ctypes.c_int64, f32p, ctypes.POINTER(ctypes.c_int)]
        lib.oracle_q6_k_subblocks.restype = None
        lib.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        lib.oracle_f32_to_f16.restype = ctypes.c_uint16
        lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.oracle_f16_to_f32.restype = ctypes.c_float
        _lib = lib
    return _lib


def _f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim != 2:
        raise ValueError(f"expected a rank-2 matrix, got shape {x.shape}")
    return x


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def quantize_q4_k(x: np.ndarray) -> np.ndarray:
    """fp32 [R, K] -> uint8 [R, K/256*144] (vulkan.py:188-419)."""
    x = _f32(x)
    rows, k = x.shape
    if k % 256:
        raise ValueError(f"Q4_K needs K % 256 == 0, got {k}")
    out = np.empty((rows, k // 256 * Q4_K_BLOCK_BYTES), dtype=np.uint8)
    _load().oracle_quantize_q4_k(_ptr(x, ctypes.c_float), rows, k, _ptr(out, ctypes.c_uint8))
    return out


def quantize_q6_k(x: np.ndarray) -> np.ndarray:
    """fp32 [R, K] -> uint8 [R, K/256*210] (vulkan.py:422-636)."""
    x = _f32(x)
    rows, k = x.shape
    if k % 256:
        raise ValueError(f"Q6_K needs K % 256 == 0, got {k}")
    out = np.empty((rows, k // 256 * Q6_K_BLOCK_BYTES), dtype=np.uint8)
    _load().oracle_quantize_q6_k(_ptr(x, ctypes.c_float), rows, k, _ptr(out, ctypes.c_uint8))
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """fp32 [R, K] -> uint8 [R, ceil(K/32)*34]; K is zero-padded to 32 as gguf.py:125-127 declares."""
    x = _f32(x)
    rows, k = x.shape
    padded = (k + 31) // 32 * 32
    if padded != k:
        x = np.ascontiguousarray(np.pad(x, ((0, 0), (0, padded - k))))
    out = np.empty((rows, padded // 32 * Q8_0_BLOCK_BYTES), dtype=np.uint8)
    _load().oracle_quantize_q8_0(_ptr(x, ctypes.c_float), rows, padded, _ptr(out, ctypes.c_uint8))
    return out


def q4_k_subblock_search(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The Q4_K sub-block search alone (choose_subblock_scale, vulkan.py:263-329) over rows of 32 values:
    fp32 (scale, min_offset) per row, before the superblock's 6-bit coding."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 32)
    scale = np.empty(x.shape[0], np.float32)
    mins = np.empty(x.shape[0], np.float32)
    _load().oracle_q4_k_subblocks(_ptr(x, ctypes.c_float), x.shape[0], _ptr(scale, ctypes.c_float),
                                  _ptr(mins, ctypes.c_float))
    return scale, mins


def q6_k_subblock_search(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The Q6_K sub-block search alone (make_qx_quants16, vulkan.py:483-540) over rows of 16 values: the fp32
    scale and the 6-bit levels (0..63) per row, before the superblock's int8 scale coding."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 16)
    scale = np.empty(x.shape[0], np.float32)
    levels = np.empty((x.shape[0], 16), np.int32)
    _load().oracle_q6_k_subblocks(_ptr(x, ctypes.c_float), x.shape[0], _ptr(scale, ctypes.c_float),
                                  _ptr(levels, ctypes.c_int))
    return scale, levels


def _dequant(fn_name: str, w: np.ndarray, k: int, block: int, nbytes: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    rows = w.shape[0]
    if w.shape[1] != k // block * nbytes:
        raise ValueError(f"packed width {w.shape[1]} does not match K={k}")
    out = np.empty((rows, k), dtype=np.float32)
    getattr(_load(), fn_name)(_ptr(w, ctypes.c_uint8), rows, k, _ptr(out, ctypes.c_float))
    return out


def dequant_q4_k(w: np.ndarray, k: int) -> np.ndarray:
    return _dequant("oracle_dequant_q4_k", w, k, 256, Q4_K_BLOCK_BYTES)


def dequant_q6_k(w: np.ndarray, k: int) -> np.ndarray:
    return _dequant("oracle_dequant_q6_k", w, k, 256, Q6_K_BLOCK_BYTES)


def dequant_q8_0(w: np.ndarray, k: int) -> np.ndarray:
    padded = (k + 31) // 32 * 32
    return _dequant("oracle_dequant_q8_0", w, padded, 32, Q8_0_BLOCK_BYTES)[:, :k]


def f32_to_f16_bits(value: float) -> int:
    return int(_load().oracle_f32_to_f16(ctypes.c_float(value)))


def f16_bits_to_f32(bits: int) -> float:
    return float(_load().oracle_f16_to_f32(ctypes.c_uint16(bits)))


# --------------------------------------------------------------------------
# Independent numpy restatements of the reference's decoders.  Each returns
# (d, dmin, scale_codes[8], min_codes[8], nibbles[256]) per superblock, read
# with the bit arithmetic of one reference kernel.
# --------------------------------------------------------------------------


def _blocks(w: np.ndarray, nbytes: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    return w.reshape(-1, nbytes)


def decode_q4_k_gemv_style(w: np.ndarray):
    """Codes as the decode GEMV reads them: three u16 loads and 32-bit masks.

    /root/reference/src/models/optimized_qwen3/shaders/linear_nobias_q4_k_matvec_f32.py:107-160
    """
    b = _blocks(w, Q4_K_BLOCK_BYTES).astype(np.uint32)
    words = b[:, 0:144].reshape(-1, 36, 4)
    words = words[:, :, 0] | (words[:, :, 1] << 8) | (words[:, :, 2] << 16) | (words[:, :, 3] << 24)
    dm = words[:, 0]
    d = (dm & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32)
    dmin = (dm >> 16).astype(np.uint16).view(np.float16).astype(np.float32)
    sc = np.zeros((b.shape[0], 8), np.uint32)
    mn = np.zeros((b.shape[0], 8), np.uint32)

    def u16(half_index):
        off = 4 + half_index * 2
        return b[:, off] | (b[:, off + 1] << 8)

    for v_im in (0, 1):
        scale0 = u16(v_im)
        scale4 = u16(v_im + 2)
        scale8 = u16(v_im + 4)
        l = (scale4 << 16) | scale0
        h = (l & 0xC0C0C0C0) >> 2
        lf = l & 0x3F3F3F3F
        s8 = (((scale8 << 12) | scale8) & 0x0F0F0F0F) | h
        unpack = lambda v: [(v >> (8 * i)) & 255 for i in range(4)]  # noqa: E731
        sc0, sc1, sc2, sc3 = unpack(lf)
        sc4, sc5, sc6, sc7 = unpack(s8)
        # In the kernel: sc0/sc1 scale sub-blocks 2*v_im, 2*v_im+1; sc2/sc3 are their mins;
        # sc4/sc5 scale sub-blocks 2*v_im+4, +5; sc6/sc7 are their mins.
        sc[:, 2 * v_im], sc[:, 2 * v_im + 1] = sc0, sc1
        mn[:, 2 * v_im], mn[:, 2 * v_im + 1] = sc2, sc3
        sc[:, 2 * v_im + 4], sc[:, 2 * v_im + 5] = sc4, sc5
        mn[:, 2 * v_im + 4], mn[:, 2 * v_im + 5] = sc6, sc7
    # nibbles: qs word at q_offset/4 (lo nibbles -> first 32 of a 64 group, hi -> next 32)
    qs = b[:, 16:144]
    q = np.zeros((b.shape[0], 256), np.uint32)
    for group in range(4):
        byte = qs[:, group * 32:(group + 1) * 32]
        q[:, group * 64:group * 64 + 32] = byte & 0x0F
        q[:, group * 64 + 32:group * 64 + 64] = (byte >> 4) & 0x0F
    return d, dmin, sc, mn, q


def decode_q4_k_embedding_style(w: np.ndarray):
    """Codes via q4k_scale_min with its index/mask tables.

    /root/reference/src/models/quantized_qwen3/shaders/embedding_q4_k_f32.py:79-110
    """
    b = _blocks(w, Q4_K_BLOCK_BYTES).astype(np.uint32)
    d = (b[:, 0] | (b[:, 1] << 8)).astype(np.uint16).view(np.float16).astype(np.float32)
    dmin = (b[:, 2] | (b[:, 3] << 8)).astype(np.uint16).view(np.float16).astype(np.float32)
    sc = np.zeros((b.shape[0], 8), np.uint32)
    mn = np.zeros((b.shape[0], 8), np.uint32)
    for sub in range(8):
        lo = sub < 4
        scidx0 = sub if lo else sub + 4
        scidx1 = sub if lo else sub - 4
        scmask1, scshift1 = (0x30, 0) if lo else (0xC0, 2)
        mbidx0 = sub + 4
        mbidx1 = sub + 4 if lo else sub
        mbmask0, mbshift0 = (0x0F, 0) if lo else (0xF0, 4)
        mbmask1, mbshift1 = (0x30, 0) if lo else (0xC0, 2)
        sc[:, sub] = (b[:, 4 + scidx0] & 0x0F) | ((b[:, 4 + scidx1] & scmask1) >> scshift1)
        mn[:, sub] = ((b[:, 4 + mbidx0] & mbmask0) >> mbshift0) | ((b[:, 4 + mbidx1] & mbmask1) >> mbshift1)
    q = np.zeros((b.shape[0], 256), np.uint32)
    for local in range(256):
        off = (local >> 6) * 32 + (local & 31)
        byte = b[:, 16 + off]
        q[:, local] = (byte & 15) if (local & 32) == 0 else (byte >> 4)
    return d, dmin, sc, mn, q


def decode_q4_k_gemm_style(w: np.ndarray):
    """Codes via the prefill GEMM's q4k_scale_min / q4k_quant4.

    /root/reference/src/models/quantized_qwen3/shaders/linear_nobias_q4_k_f32.py:121-140
    """
    b = _blocks(w, Q4_K_BLOCK_BYTES).astype(np.uint32)
    d = (b[:, 0] | (b[:, 1] << 8)).astype(np.uint16).view(np.float16).astype(np.float32)
    dmin = (b[:, 2] | (b[:, 3] << 8)).astype(np.uint16).view(np.float16).astype(np.float32)
    sc = np.zeros((b.shape[0], 8), np.uint32)
    mn = np.zeros((b.shape[0], 8), np.uint32)
    for sub in range(8):
        if sub < 4:
            sc[:, sub] = b[:, 4 + sub] & 63
            mn[:, sub] = b[:, 8 + sub] & 63
        else:
            local = sub - 4
            d_byte, m_byte, packed = b[:, 4 + local], b[:, 8 + local], b[:, 12 + local]
            sc[:, sub] = (packed & 15) | ((d_byte >> 2) & 48)
            mn[:, sub] = (packed >> 4) | ((m_byte >> 2) & 48)
    q = np.zeros((b.shape[0], 256), np.uint32)
    for local_k in range(0, 256, 4):
        pair = local_k >> 6
        byte_index = local_k & 31
        base = 16 + pair * 32 + byte_index
        word = b[:, base] | (b[:, base + 1] << 8) | (b[:, base + 2] << 16) | (b[:, base + 3] << 24)
        word = (word & 0x0F0F0F0F) if (local_k & 32) == 0 else ((word >> 4) & 0x0F0F0F0F)
        for j in range(4):
            q[:, local_k + j] = (word >> (8 * j)) & 0xFF
    return d, dmin, sc, mn, q


def q4_k_values_from_codes(d, dmin, sc, mn, q) -> np.ndarray:
    """d*sc*q - dmin*m in fp32 with the embedding decoder's operation order."""
    d = d.astype(np.float32)[:, None]
    dmin = dmin.astype(np.float32)[:, None]
    scale = np.repeat(sc.astype(np.float32), 32, axis=1)
    mins = np.repeat(mn.astype(np.float32), 32, axis=1)
    return (d * scale) * q.astype(np.float32) - dmin * mins


def decode_q6_k_codes(w: np.ndarray):
    """(d, int8 scales[16], q-32 in [-32,31] [256]) via the K6/K26 word-level decoder.

    /root/reference/src/models/quantized_qwen3/shaders/linear_nobias_q6_k_matvec_f32.py:116-156
    """
    b = _blocks(w, Q6_K_BLOCK_BYTES).astype(np.uint32)
    d = (b[:, 208] | (b[:, 209] << 8)).astype(np.uint16).view(np.float16).astype(np.float32)
    scales = b[:, 192:208].astype(np.uint8).view(np.int8).astype(np.int32)
    q = np.zeros((b.shape[0], 256), np.int32)

    def u32(off):
        return b[:, off] | (b[:, off + 1] << 8) | (b[:, off + 2] << 16) | (b[:, off + 3] << 24)

    for itid in range(16):
        v_im = itid >> 3
        v_in = itid - 8 * v_im
        l0 = 4 * v_in
        ql0 = u32(64 * v_im + l0)
        ql32 = u32(64 * v_im + l0 + 32)
        qh = u32(128 + 32 * v_im + l0)
        words = [
            (ql0 & 0x0F0F0F0F) | ((qh & 0x03030303) << 4),
            (ql32 & 0x0F0F0F0F) | ((qh & 0x0C0C0C0C) << 2),
            ((ql0 >> 4) & 0x0F0F0F0F) | (qh & 0x30303030),
            ((ql32 >> 4) & 0x0F0F0F0F) | ((qh & 0xC0C0C0C0) >> 2),
        ]
        for part, word in enumerate(words):
            for j in range(4):
                q[:, 128 * v_im + 32 * part + l0 + j] = ((word >> (8 * j)) & 0xFF).astype(np.int32) - 32
    return d, scales, q


def decode_q8_0_codes(w: np.ndarray):
    """(d, int8 q[32]) per block (linear_nobias_q8_0_matvec_f32.py:84-95)."""
    b = _blocks(w, Q8_0_BLOCK_BYTES)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
    q = b[:, 2:34].view(np.int8).astype(np.int32)
    return d, q
