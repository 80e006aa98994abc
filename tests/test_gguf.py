"""GGUF reader, writer, Q4_K_M policy and the Qwen3 loader (torch2vk_amd.gguf).

The format is pinned by a file assembled here byte by byte from the public GGUF v3 layout (independently of
the writer): the reader must parse it and the writer must reproduce it exactly.  The reference holds no GGUF
fixture (its tests need HF checkpoints), so the policy is pinned by the reference's own rule
(src/torch2vk/quantize/gguf.py:54-83, src/models/quantized_qwen3/quantization.py:17-32) on Qwen3 names.
"""

from __future__ import annotations

import struct
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import quant
from torch2vk_amd import gguf
from torch2vk_amd.gguf import GGUFMetadataValue as MV
from torch2vk_amd.gguf import GGUFTensor, GGUFTensorType as T, GGUFValueType as V


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _pad(b: bytes, align: int = 32) -> bytes:
    return b + bytes(-len(b) % align)


def _hand_file() -> tuple[bytes, dict, list]:
    """A two-tensor GGUF v3 file written out field by field."""
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    q8 = np.frombuffer(bytes(range(34)), dtype=np.uint8).reshape(1, 34)
    kv = (_str("general.architecture") + struct.pack("<I", 8) + _str("qwen3")
          + _str("general.file_type") + struct.pack("<II", 4, 15)
          + _str("t.f32") + struct.pack("<If", 6, 1.5)
          + _str("t.arr") + struct.pack("<IIQ", 9, 5, 3) + struct.pack("<iii", -1, 0, 7)
          + _str("t.bool") + struct.pack("<IB", 7, 1))
    infos = (_str("a") + struct.pack("<I", 2) + struct.pack("<QQ", 3, 2) + struct.pack("<IQ", 0, 0)
             + _str("b") + struct.pack("<I", 2) + struct.pack("<QQ", 32, 1) + struct.pack("<IQ", 8, 32))
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, 5) + kv + infos
    data = _pad(a.tobytes()) + _pad(q8.tobytes())
    meta = [MV("general.architecture", V.STRING, "qwen3"), MV("general.file_type", V.UINT32, 15),
            MV("t.f32", V.FLOAT32, 1.5), MV("t.arr", V.ARRAY, [-1, 0, 7], V.INT32), MV("t.bool", V.BOOL, True)]
    tensors = [GGUFTensor("a", T.F32, (2, 3), a), GGUFTensor("b", T.Q8_0, (1, 32), q8)]
    return _pad(head) + data, meta, tensors


def test_reader_parses_hand_assembled_file(tmp_path):
    raw, _, tensors = _hand_file()
    p = tmp_path / "hand.gguf"
    p.write_bytes(raw)
    with gguf.open_gguf_mmap(p) as g:
        assert g.metadata["GGUF.version"] == 3
        assert g.metadata["general.architecture"] == "qwen3"
        assert g.metadata["general.file_type"] == 15
        assert g.metadata["t.f32"] == 1.5 and g.metadata["t.arr"] == [-1, 0, 7] and g.metadata["t.bool"] is True
        ea, eb = g.entry("a"), g.entry("b")
        assert ea.ggml_shape == (3, 2) and ea.logical_shape == (2, 3) and ea.nbytes == 24
        assert eb.ggml_type is T.Q8_0 and eb.logical_shape == (1, 32) and eb.nbytes == 34
        assert ea.data_offset % 32 == 0 and eb.data_offset == ea.data_offset + 32
        np.testing.assert_array_equal(g.float_array("a"), tensors[0].data)
        np.testing.assert_array_equal(g.array("b"), tensors[1].data)
        assert bytes(g.buffer_rows("a", row_offset=1, row_count=1)) == tensors[0].data[1].tobytes()


def test_writer_reproduces_hand_assembled_file(tmp_path):
    raw, meta, tensors = _hand_file()
    p = gguf.write_gguf(tmp_path / "w.gguf", meta, tensors)
    assert p.read_bytes() == raw


def test_round_trip_quantized_types_and_alignment(tmp_path):
    rng = np.random.default_rng(0)
    w4 = quant.quantize_q4_k(rng.standard_normal((3, 512)).astype(np.float32))
    w6 = quant.quantize_q6_k(rng.standard_normal((2, 256)).astype(np.float32))
    w8 = quant.quantize_q8_0(rng.standard_normal((5, 64)).astype(np.float32))
    f16 = rng.standard_normal(7).astype(np.float16)
    tensors = [GGUFTensor("w4", T.Q4_K, (3, 512), w4), GGUFTensor("w6", T.Q6_K, (2, 256), w6),
               GGUFTensor("w8", T.Q8_0, (5, 64), w8), GGUFTensor("n", T.F16, (7,), f16)]
    meta = {"general.alignment": 64, "general.name": "t", "x.u64": MV("x.u64", V.UINT64, 2**40),
            "x.floats": [0.5, 2.0]}
    p = gguf.write_gguf(tmp_path / "r.gguf", meta, tensors)
    with gguf.open_gguf_mmap(p) as g:
        assert g.metadata["general.alignment"] == 64 and g.metadata["x.u64"] == 2**40
        assert g.metadata["x.floats"] == [0.5, 2.0]
        for t in tensors:
            e = g.entry(t.name)
            assert e.data_offset % 64 == 0 and e.ggml_type is t.ggml_type and e.logical_shape == t.logical_shape
        np.testing.assert_array_equal(g.array("w4"), w4)
        np.testing.assert_array_equal(g.array("w6"), w6)
        np.testing.assert_array_equal(g.array("w8"), w8)
        np.testing.assert_array_equal(g.float_array("n"), f16.astype(np.float32))
        assert g.entry("w4").row_bytes == 2 * 144 and g.entry("w6").row_bytes == 210


def test_rejects_bad_files(tmp_path):
    raw, _, _ = _hand_file()
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUX" + raw[4:])
    with pytest.raises(ValueError, match="not a GGUF"):
        gguf.read_gguf_index(p)
    p.write_bytes(raw[:4] + struct.pack("<I", 1) + raw[8:])
    with pytest.raises(ValueError, match="version"):
        gguf.read_gguf_index(p)
    p.write_bytes(raw[:60])
    with pytest.raises(ValueError, match="truncated"):
        gguf.read_gguf_index(p)
    with pytest.raises(ValueError, match="blocks"):
        GGUFTensor("x", T.Q4_K, (1, 100), np.zeros(0, np.uint8))
    with pytest.raises(ValueError, match="needs"):
        GGUFTensor("x", T.Q4_K, (1, 256), np.zeros(143, np.uint8))


def test_q4_k_m_policy_on_qwen3_names():
    L = 28
    cfg = gguf.qwen3_q4_k_m_config(L)
    more = {0, 1, 2, 5, 8, 11, 14, 17, 20, 23, 24, 25, 26, 27}  # i < 3, i >= 24, (i - 3) % 3 == 2
    for i in range(L):
        v = cfg.gguf_type(checkpoint_key=f"model.layers.{i}.self_attn.v_proj.weight", shape=(1024, 1024))
        d = cfg.gguf_type(checkpoint_key=f"model.layers.{i}.mlp.down_proj.weight", shape=(1024, 3072))
        q = cfg.gguf_type(checkpoint_key=f"model.layers.{i}.self_attn.q_proj.weight", shape=(2048, 1024))
        assert (v, d) == ((T.Q6_K, T.Q6_K) if i in more else (T.Q4_K, T.Q4_K)), i
        assert q is T.Q4_K
    assert cfg.gguf_type(checkpoint_key="lm_head.weight", shape=(151936, 1024)) is T.Q6_K
    assert cfg.gguf_type(checkpoint_key="model.embed_tokens.weight", shape=(151936, 1024)) is T.Q4_K
    assert cfg.gguf_type(checkpoint_key="model.norm.weight", shape=(1024,)) is T.F32
    assert cfg.gguf_type(checkpoint_key="x", shape=(4, 96)) is T.Q8_0          # K % 32 only
    assert cfg.gguf_type(checkpoint_key="x", shape=(4, 100)) is T.F32
    assert cfg.gguf_type(checkpoint_key="x", shape=(4, 256), dtype="int64") is T.F32
    assert replace(cfg, f16_tensor_prefixes=("x",)).gguf_type(checkpoint_key="xy", shape=(4, 256)) is T.F16
    assert replace(cfg, q8_tensor_names=("lm_head.weight",)).gguf_type(
        checkpoint_key="lm_head.weight", shape=(8, 256)) is T.Q8_0            # Q8 wins over Q6
    md = {m.key: m.value for m in cfg.metadata()}
    assert md["general.architecture"] == "qwen3" and md["general.file_type"] == 15


def _tiny_qwen3():
    from torch2vk_amd.qwen3.config import Qwen3Config

    # hidden 1024: the Q6_K GEMV serves rows of 1024 values and more (Q4_K_M puts layer 1's v/down and the
    # LM head in Q6_K)
    return Qwen3Config("tiny", hidden=1024, layers=2, heads=8, kv_heads=4, head_dim=128, mlp=2048, vocab=384,
                       eos_token_ids=(383,))


def _tiny_checkpoint(cfg, seed=0, tied=False) -> dict[str, np.ndarray]:
    from torch2vk_amd.qwen3.weights import matrix_shapes, norm_shapes

    rng = np.random.default_rng(seed)
    inv = {v: k for k, v in gguf.qwen3_tensor_names(cfg.layers).items()}
    ck = {}
    for key, shape in matrix_shapes(cfg).items():
        if tied and key == "lm_head":
            continue
        ck[inv[key]] = (rng.standard_normal(shape) * 0.05).astype(np.float32)
    for key, n in norm_shapes(cfg).items():
        ck[inv[key]] = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    return ck


def _oracle_gguf(path, ck: dict[str, np.ndarray], cfg_policy) -> None:
    """A GGUF file of ``ck`` quantized by the CPU oracle under ``cfg_policy`` (test-side writer)."""
    fn = {T.Q4_K: quant.quantize_q4_k, T.Q6_K: quant.quantize_q6_k, T.Q8_0: quant.quantize_q8_0}
    tensors = []
    for name, a in ck.items():
        t = cfg_policy.gguf_type(checkpoint_key=name, shape=a.shape)
        data = fn[t](a) if t in fn else a
        tensors.append(GGUFTensor(name, t, a.shape, data))
    gguf.write_gguf(path, cfg_policy.metadata(), tensors)


@pytest.mark.parametrize("tied", [False, True])
def test_load_qwen3_gguf_on_cpu(tmp_path, tied):
    cfg = _tiny_qwen3()
    ck = _tiny_checkpoint(cfg, tied=tied)
    policy = gguf.qwen3_q4_k_m_config(cfg.layers)
    _oracle_gguf(tmp_path / "m.gguf", ck, policy)
    w = gguf.load_qwen3_gguf(tmp_path / "m.gguf", cfg, device="cpu")
    names = gguf.qwen3_tensor_names(cfg.layers)
    for ck_name, key in names.items():
        if key in w.packed:
            src_name = "model.embed_tokens.weight" if (tied and key == "lm_head") else ck_name
            src = ck[src_name]
            want_t = policy.gguf_type(checkpoint_key=src_name, shape=src.shape)
            assert w.types[key] == gguf.KERNEL_TYPE[want_t], key
            fn = {"q4_k": quant.quantize_q4_k, "q6_k": quant.quantize_q6_k, "q8_0": quant.quantize_q8_0}
            np.testing.assert_array_equal(w.packed[key].numpy(), fn[w.types[key]](src), err_msg=key)
        else:
            np.testing.assert_array_equal(w.norms[key].numpy(), ck[ck_name])
    # q, k, v of a layer share one allocation (the persistent kernel streams them as one matrix)
    for i in range(cfg.layers):
        q, k, v = (w.packed[f"layers.{i}.{n}"] for n in ("q", "k", "v"))
        if len({w.types[f"layers.{i}.{n}"] for n in ("q", "k", "v")}) == 1:
            assert k.data_ptr() == q.data_ptr() + q.numel() and v.data_ptr() == k.data_ptr() + k.numel()


def test_load_rejects_mismatched_config(tmp_path):
    cfg = _tiny_qwen3()
    _oracle_gguf(tmp_path / "m.gguf", _tiny_checkpoint(cfg), gguf.qwen3_q4_k_m_config(cfg.layers))
    with pytest.raises(ValueError, match="shape"):
        gguf.load_qwen3_gguf(tmp_path / "m.gguf", replace(cfg, mlp=2304), device="cpu")
    with pytest.raises(KeyError):
        gguf.load_qwen3_gguf(tmp_path / "m.gguf", replace(cfg, layers=3), device="cpu")


@pytest.mark.gpu
def test_export_load_decode_matches_oracle(device, tmp_path):
    """safetensors -> export_q4_k_m_gguf (GPU quantizers) -> bytes equal the oracle quantizers' -> load ->
    greedy decode on the GPU equals the CPU oracle decoder's tokens."""
    from safetensors.torch import save_file

    from oracle.qwen3_check import check_greedy_tokens, decoder_step_logits, dense_weights
    from oracle.reference import Qwen3Shape
    from torch2vk_amd.qwen3.model import Qwen3Decoder
    from torch2vk_amd.qwen3.weights import matrix_shapes

    cfg = _tiny_qwen3()
    ck = _tiny_checkpoint(cfg, seed=3)
    (tmp_path / "ck").mkdir()
    save_file({k: torch.from_numpy(v) for k, v in ck.items()}, str(tmp_path / "ck" / "model.safetensors"))
    policy = gguf.qwen3_q4_k_m_config(cfg.layers)
    print("export tiny Qwen3 checkpoint to GGUF", flush=True)
    out = gguf.export_q4_k_m_gguf(model_dir=tmp_path / "ck", output=tmp_path / "m.gguf", config=policy)
    _oracle_gguf(tmp_path / "ref.gguf", ck, policy)
    with gguf.open_gguf_mmap(out) as a, gguf.open_gguf_mmap(tmp_path / "ref.gguf") as b:
        assert set(a.tensors) == set(b.tensors)
        for n in a.tensors:
            assert a.entry(n).ggml_type is b.entry(n).ggml_type, n
            np.testing.assert_array_equal(np.asarray(a.array(n)), np.asarray(b.array(n)), err_msg=n)
    assert gguf.export_q4_k_m_gguf(model_dir=tmp_path / "ck", output=out, config=policy) == out  # kept
    w = gguf.load_qwen3_gguf(out, cfg, device=device)
    dec = Qwen3Decoder(w, max_positions=64, max_new_tokens=8)
    dec.stop_on_eos = False
    prompt = [5, 17, 200, 3]
    tokens = dec.generate(torch.tensor(prompt, dtype=torch.int64, device=device), 8)
    dense = dense_weights({k: v.cpu().numpy() for k, v in w.packed.items()}, w.types,
                          {k: v.cpu().numpy() for k, v in w.norms.items()}, matrix_shapes(cfg))
    shape = Qwen3Shape(hidden=cfg.hidden, layers=cfg.layers, heads=cfg.heads, kv_heads=cfg.kv_heads,
                       head_dim=cfg.head_dim, mlp=cfg.mlp, vocab=cfg.vocab, rope_theta=cfg.rope_theta)
    print(check_greedy_tokens(shape, dense, prompt, tokens, kv_history=(dec.k_cache, dec.v_cache),
                              gpu_logits=decoder_step_logits(dec), label="gguf"))
