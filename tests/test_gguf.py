"""GGUF ingestion (qmoe_gguf_* over the C ABI, qwenium_amd.gguf).

The reader follows the reference's loader (src/loader/gguf_loader.cpp:46-91
header, 245-436 metadata, 474-497 inventory, 84-85 data alignment, 621-639
tensor data).  Pins:
  * a hand-assembled byte string whose every offset is written out below;
  * round trips through an independent writer (tests/gguf_writer.py) with
    every metadata value type, string arrays and three tensor types;
  * every failure the reference's loader raises (magic, version, truncation,
    data past the end of the file, missing tensor) plus the typed lookups;
  * on the GPU: a layer built from a GGUF file gives the bits of the same
    layer built from the same bytes in memory (whose parity with the oracle
    is pinned in test_gpu_parity.py).
"""
import struct

import numpy as np
import pytest

from qwenium_amd import gguf as G
from qwenium_amd._lib import (QMOE_ERR_CAPACITY, QMOE_ERR_TYPE, QMOE_ERR_VALUE, QmoeError, TYPE_F32, TYPE_Q4_0,
                              TYPE_Q8_0)
import gguf_writer as W


def test_hand_assembled_minimal_file(tmp_path):
    # header (24 B) | 1 KV: key "general.architecture" (8 + 20), type 8 (4), "qwen35moe" (8 + 9)
    # | 1 tensor: name "t" (8 + 1), n_dims 1 (4), ne[0] = 2 (8), type 0 (4), offset 0 (8)
    # = 24 + 28 + 4 + 17 + 9 + 4 + 8 + 4 + 8 = 106 -> data at 128 (32-byte alignment)
    b = struct.pack("<IIQQ", 0x46554747, 3, 1, 1)
    b += struct.pack("<Q", 20) + b"general.architecture" + struct.pack("<I", 8) + struct.pack("<Q", 9) + b"qwen35moe"
    b += struct.pack("<Q", 1) + b"t" + struct.pack("<I", 1) + struct.pack("<Q", 2) + struct.pack("<IQ", 0, 0)
    assert len(b) == 106
    b += b"\0" * (128 - len(b)) + struct.pack("<ff", 1.5, -2.25)
    p = tmp_path / "min.gguf"
    p.write_bytes(b)
    with G.GGUFFile(str(p)) as f:
        assert f.info() == {"version": 3, "n_tensors": 1, "n_kv": 1, "data_offset": 128}
        assert f.get_str("general.architecture") == "qwen35moe"
        t = f.find("t")
        assert (t.type, t.n_dims, t.ne[0], t.file_offset, t.nbytes) == (0, 1, 2, 128, 8)
        assert struct.unpack("<ff", f.read("t")) == (1.5, -2.25)


def _kv_all_types():
    return [
        ("general.architecture", W.STR, "qwen35moe"),
        ("general.name", W.STR, "tiny ünïcode"),
        ("k.u8", W.U8, 200), ("k.i8", W.I8, -5), ("k.u16", W.U16, 60000), ("k.i16", W.I16, -30000),
        ("k.u32", W.U32, 4000000000), ("k.i32", W.I32, -7), ("k.f32", W.F32, 1e-6), ("k.bool", W.BOOL, True),
        ("k.u64", W.U64, 1 << 40), ("k.i64", W.I64, -(1 << 40)), ("k.f64", W.F64, 0.1),
        ("tokenizer.ggml.tokens", W.ARR, (W.STR, ["a", "bc", "", "déf"])),
        ("k.arr_u32", W.ARR, (W.U32, [1, 2, 3])),
        ("k.arr_f64", W.ARR, (W.F64, [0.5, 0.25])),
        ("qwen35moe.expert_count", W.U32, 4),
        ("qwen35moe.expert_used_count", W.U32, 2),
        ("qwen35moe.expert_feed_forward_length", W.U32, 64),
    ]


def _tensors(rng):
    f32 = rng.standard_normal((3, 4)).astype(np.float32)        # ne (4, 3)
    q8 = rng.integers(0, 256, size=2 * 2 * 34, dtype=np.uint8)  # ne (64, 2): 2 rows of 2 blocks
    q4 = rng.integers(0, 256, size=3 * 2 * 18, dtype=np.uint8)  # ne (32, 3, 2): 6 rows of 1 block
    return [("a.f32", TYPE_F32, (4, 3), f32.tobytes()), ("b.q8", TYPE_Q8_0, (64, 2), q8.tobytes()),
            ("c.q4", TYPE_Q4_0, (32, 3, 2), q4.tobytes())]


@pytest.mark.parametrize("alignment", [32, 64])
def test_round_trip_metadata_and_tensors(tmp_path, alignment):
    rng = np.random.default_rng(0)
    kv = _kv_all_types()
    if alignment != 32:
        kv.append(("general.alignment", W.U32, alignment))
    tens = _tensors(rng)
    p = tmp_path / "rt.gguf"
    blob = W.write_gguf(str(p), kv, tens, alignment=alignment)
    with G.GGUFFile(str(p)) as f:
        info = f.info()
        assert info["version"] == 3 and info["n_tensors"] == 3 and info["n_kv"] == len(kv)
        assert info["data_offset"] % alignment == 0
        assert f.get_str("general.name") == "tiny ünïcode"
        assert f.get_u32("k.u32") == 4000000000
        assert f.get_f32("k.f32") == np.float32(1e-6)
        assert f.tensor_names() == ["a.f32", "b.q8", "c.q4"]
        for name, gtype, ne, data in tens:
            t = f.find(name)
            assert t.type == gtype and t.n_dims == len(ne)
            assert tuple(t.ne[d] for d in range(len(ne))) == ne
            assert t.nbytes == len(data)
            assert t.file_offset % alignment == 0
            assert blob[t.file_offset:t.file_offset + t.nbytes] == data
            assert f.read(name) == data
        assert f.moe_hparams() == G.Hparams(4, 2, 64, False)


def test_typed_lookups_fail_loud(tmp_path):
    p = tmp_path / "kv.gguf"
    W.write_gguf(str(p), _kv_all_types(), [])
    with G.GGUFFile(str(p)) as f:
        for call, key, msg in [(f.get_u32, "k.i32", 'key "k.i32" expected type UINT32, got type 5'),
                               (f.get_f32, "k.f64", 'key "k.f64" expected type FLOAT32, got type 12'),
                               (f.get_str, "k.u8", 'key "k.u8" expected type STRING, got type 0'),
                               (f.get_u32, "nope", 'key "nope" expected present, got absent')]:
            with pytest.raises(QmoeError) as e:
                call(key)
            assert e.value.code == QMOE_ERR_VALUE and msg in str(e.value)
        with pytest.raises(QmoeError, match='tensor "missing" expected present, got absent'):
            f.find("missing")


@pytest.mark.parametrize("case", ["magic", "version4", "version1", "truncated_header", "truncated_kv",
                                  "truncated_inventory", "bad_value_type", "bad_dims"])
def test_open_rejects_malformed_files(tmp_path, case):
    kv = [("general.architecture", W.STR, "qwen35moe"), ("k", W.U32, 1)]
    tens = [("t", TYPE_F32, (4,), b"\0" * 16)]
    b = W.gguf_bytes(kv, tens)
    want = {
        "magic": "invalid magic number",
        "version4": "unsupported GGUF version: expected 2 or 3, got 4",
        "version1": "unsupported GGUF version: expected 2 or 3, got 1",
        "truncated_header": "too small for the GGUF header",
        "truncated_kv": "read past end of file",
        "truncated_inventory": "read past end of file",
        "bad_value_type": "unknown metadata value type 13",
        "bad_dims": "expected 1..4 dims, got 5",
    }[case]
    if case == "magic":
        b = W.gguf_bytes(kv, tens, magic=0x46554748)
    elif case == "version4":
        b = W.gguf_bytes(kv, tens, version=4)
    elif case == "version1":
        b = W.gguf_bytes(kv, tens, version=1)
    elif case == "truncated_header":
        b = b[:20]
    elif case == "truncated_kv":
        b = b[:24 + 8 + 10]
    elif case == "truncated_inventory":
        inv = len(W.gguf_bytes(kv, [], alignment=1))  # header + metadata, no padding
        b = b[:inv + 8 + 1 + 4 + 3]  # inside the tensor's ne
    elif case == "bad_value_type":
        b = struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13)
    elif case == "bad_dims":
        b = struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + struct.pack("<Q", 1) + b"t" + struct.pack("<I", 5)
    p = tmp_path / f"{case}.gguf"
    p.write_bytes(b)
    with pytest.raises(QmoeError) as e:
        G.GGUFFile(str(p))
    assert e.value.code == QMOE_ERR_VALUE
    assert want in str(e.value)


def test_tensor_data_past_end_and_unknown_type(tmp_path):
    tens = [("t", TYPE_F32, (8,), b"\0" * 32), ("u", 99, (4,), b"\0" * 4)]
    b = W.gguf_bytes([], tens)
    p = tmp_path / "short.gguf"
    p.write_bytes(b[:-8])  # u's data and the end of t's cut off
    with G.GGUFFile(str(p)) as f:
        with pytest.raises(QmoeError, match='tensor data for "t" would read past end of file'):
            f.find("t")
        with pytest.raises(QmoeError) as e:
            f.find("u")
        assert e.value.code == QMOE_ERR_TYPE


def _crafted_inventory(entries):
    """A v3 file with no metadata and the given inventory (name, ne tuple, ggml
    type, offset), data start aligned to 32 bytes, 64 bytes of data."""
    b = struct.pack("<IIQQ", 0x46554747, 3, len(entries), 0)
    for name, ne, typ, off in entries:
        b += struct.pack("<Q", len(name)) + name + struct.pack("<I", len(ne))
        b += b"".join(struct.pack("<Q", v % 2**64) for v in ne) + struct.pack("<IQ", typ, off % 2**64)
    b += b"\0" * (-len(b) % 32)
    return b, len(b), b + bytes(range(64))


def test_crafted_sizes_and_offsets_do_not_wrap(tmp_path):
    """An element count or byte size past 64 bits, or a data offset whose sum with the
    data start wraps, is rejected instead of aliasing other bytes of the file
    (the reference bounds-checks the tensor data, gguf_loader.cpp:621-639)."""
    entries = [
        (b"a", (2**62, 4), TYPE_F32, 0),      # 2^64 elements: wraps to 0 bytes
        (b"b", (2**61 + 1, 8), TYPE_F32, 0),  # 2^64 + 8 elements: wraps to 32 bytes
        (b"c", (2**62 + 2,), TYPE_F32, 0),    # 2^62 + 2 elements fit, their bytes wrap to 8
        (b"d", (2,), TYPE_F32, 0),
    ]
    start = _crafted_inventory(entries)[1]  # the data start (offsets do not change the layout)
    entries[3] = (b"d", (2,), TYPE_F32, 2**64 - start + 8)  # data start + offset wraps to byte 8
    b = _crafted_inventory(entries)[2]
    assert 8 + 8 <= len(b)  # a wrapped read would land inside the file
    p = tmp_path / "crafted.gguf"
    p.write_bytes(b)
    with G.GGUFFile(str(p)) as f:
        for name in ("a", "b", "c"):
            with pytest.raises(QmoeError, match=f'tensor "{name}" expected a shape whose byte size fits 64 bits'):
                f.find(name)
        with pytest.raises(QmoeError, match='tensor data for "d" would read past end of file'):
            f.find("d")


def test_read_buffer_too_small(tmp_path):
    import ctypes

    from qwenium_amd._lib import lib

    p = tmp_path / "rb.gguf"
    W.write_gguf(str(p), [], [("t", TYPE_F32, (8,), b"\1" * 32)])
    with G.GGUFFile(str(p)) as f:
        buf = ctypes.create_string_buffer(16)
        rc = lib().qmoe_gguf_read(f._handle, b"t", buf, 16)
        assert rc == QMOE_ERR_CAPACITY


def test_tensor_view_strides():
    t = G.QmoeGgufTensor()
    t.type, t.n_dims = TYPE_Q4_0, 3
    for d, n in enumerate((2048, 512, 256, 1)):
        t.ne[d] = n
    v = G.tensor_view(t, 0x1000)
    assert (v.type, v.n_dims) == (TYPE_Q4_0, 3)
    assert list(v.nb) == [18, 64 * 18, 64 * 18 * 512, 64 * 18 * 512 * 256]
    t.ne[0] = 100  # not a whole number of blocks
    with pytest.raises(QmoeError):
        G.tensor_view(t, 0x1000)


def test_moe_hparams_checks(tmp_path):
    kv = [("general.architecture", W.STR, "qwen35moe"), ("qwen35moe.expert_count", W.U32, 4),
          ("qwen35moe.expert_used_count", W.U32, 5), ("qwen35moe.expert_feed_forward_length", W.U32, 64)]
    p = tmp_path / "hp.gguf"
    W.write_gguf(str(p), kv, [])
    with G.GGUFFile(str(p)) as f:
        with pytest.raises(ValueError, match=r'"expert_used_count" expected <= expert_count \(4\), got 5'):
            f.moe_hparams()


# ---------------------------------------------------------------------------
# GPU: a layer from a GGUF file == the same layer from the same bytes in memory
# ---------------------------------------------------------------------------
def _write_block_gguf(path, spec, seed, n_blocks=2):
    import torch

    from qwenium_amd import synthetic as S

    kv = [("general.architecture", W.STR, "qwen35moe"),
          ("qwen35moe.block_count", W.U32, n_blocks),
          ("qwen35moe.embedding_length", W.U32, spec.n_embd),
          ("qwen35moe.expert_count", W.U32, spec.n_experts),
          ("qwen35moe.expert_used_count", W.U32, spec.top_k),
          ("qwen35moe.expert_feed_forward_length", W.U32, spec.ffn_dim),
          ("qwen35moe.attention.layer_norm_rms_epsilon", W.F32, 1e-6)]
    tens, layers = [], []
    for blk in range(n_blocks):
        t = S.make_layer_tensors(spec, seed, layer=blk)
        layers.append(t)
        for slot, suffix in G.MOE_SLOTS:
            if slot not in t:
                continue
            g = t[slot]
            tens.append((f"blk.{blk}.{suffix}", g.type, tuple(g.ne), g.data.cpu().numpy().tobytes()))
        w = S.make_norm_weight(spec, seed, blk)
        tens.append((f"blk.{blk}.{G.FFN_NORM}", TYPE_F32, (spec.n_embd,), w.cpu().numpy().tobytes()))
    torch.cuda.synchronize()
    W.write_gguf(path, kv, tens)
    return layers


@pytest.mark.gpu
@pytest.mark.parametrize("which", ["config1", "shared_q4"])
def test_gguf_layer_matches_in_memory_layer(gpu, tmp_path, which):
    import torch

    from qwenium_amd import Workspace
    from qwenium_amd import synthetic as S

    spec = S.CONFIG1 if which == "config1" else S.LayerSpec(512, 16, 4, 128, True, TYPE_Q4_0)
    p = str(tmp_path / "model.gguf")
    tensors = _write_block_gguf(p, spec, seed=3)
    with G.GGUFFile(p) as f:
        assert f.moe_hparams(block=1) == spec.hparams
        for blk in (0, 1):
            lg = f.moe_layer(blk)
            lm = S.make_layer(spec, 3, layer=blk, tensors=tensors[blk])
            for T in (1, 10, 37):
                x = S.make_x(spec, T, seed=3, batch=T)
                ws = Workspace(lg, T)
                yg = lg.forward(x, workspace=ws)
                ym = lm.forward(x, workspace=ws)
                torch.cuda.synchronize()
                assert torch.equal(yg, ym), (blk, T)
            w = f.ffn_norm(blk)
            assert torch.equal(w, S.make_norm_weight(spec, 3, blk))


@pytest.mark.gpu
def test_gguf_gemma4_layer_matches_in_memory_layer(gpu, tmp_path):
    """A Gemma 4 block (fused ffn_gate_up_exps, gemma4.* hparams, the MoE-branch
    norms) read from a file gives the bits of the in-memory layer."""
    import torch

    from qwenium_amd import Workspace
    from qwenium_amd import synthetic as S

    spec = S.LayerSpec(512, 16, 4, 128, False, TYPE_Q4_0, geglu=True)
    kv = [("general.architecture", W.STR, "gemma4"), ("gemma4.expert_count", W.U32, spec.n_experts),
          ("gemma4.expert_used_count", W.U32, spec.top_k),
          ("gemma4.expert_feed_forward_length", W.U32, spec.ffn_dim)]
    t = S.make_layer_tensors(spec, 5)
    pre, rs = S.make_gemma4_norms(spec, 5, 0)
    tens = [(f"blk.0.{suffix}", t[slot].type, tuple(t[slot].ne), t[slot].data.cpu().numpy().tobytes())
            for slot, suffix in G.GEMMA4_MOE_SLOTS]
    tens += [(f"blk.0.{G.GEMMA4_PRE_NORM}", TYPE_F32, (spec.n_embd,), pre.cpu().numpy().tobytes()),
             (f"blk.0.{G.GEMMA4_ROUTER_SCALE}", TYPE_F32, (spec.n_embd,), rs.cpu().numpy().tobytes())]
    p = str(tmp_path / "gemma4.gguf")
    W.write_gguf(p, kv, tens)
    lm = S.make_layer(spec, 5, tensors=t)
    with G.GGUFFile(p) as f:
        lg = f.gemma4_moe_layer(0)
        pg, rg = f.gemma4_moe_norms(0)
        assert torch.equal(pg, pre) and torch.equal(rg, rs)
        for T in (1, 10, 200):
            x = S.make_x(spec, T, seed=5, batch=T)
            ws = Workspace(lg, T)
            yg = lg.forward_gemma4(x, pg, rg, 1e-6, workspace=ws)
            ym = lm.forward_gemma4(x, pre, rs, 1e-6, workspace=ws)
            torch.cuda.synchronize()
            assert torch.equal(yg, ym), T
        with pytest.raises(ValueError, match="gemma4: missing tensor 'blk.1.ffn_gate_inp.weight'"):
            f.gemma4_moe_layer(1)
