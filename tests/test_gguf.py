"""GGUF v3 container reader / writer (librtq.so, host code only: no GPU needed).

The reference commits no GGUF fixtures and the image has no GGUF library, so the pin is an image
encoded here directly from the public GGUF v3 specification with ``struct`` (independent of the
library's writer): the reader must decode it, and the writer must reproduce it byte for byte.
Round trips, every truncation of an image and malformed headers cover the rest.
"""
import os
import struct

import numpy as np
import pytest

from rust_trainer_amd import RtqError
from rust_trainer_amd import gguf as G
from rust_trainer_amd.synth import QUANTIZERS, Rng


def s_(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def spec_image(alignment=None):
    """A GGUF v3 image built by hand: 13 metadata keys over every value type, 3 tensors."""
    kvs = [
        ("general.architecture", 8, s_("qwen3")),
        ("k.u8", 0, struct.pack("<B", 200)),
        ("k.i8", 1, struct.pack("<b", -5)),
        ("k.u16", 2, struct.pack("<H", 65000)),
        ("k.i16", 3, struct.pack("<h", -300)),
        ("k.u32", 4, struct.pack("<I", 4000000000)),
        ("k.i32", 5, struct.pack("<i", -7)),
        ("adapter.lora.alpha", 6, struct.pack("<f", 8.0)),
        ("k.bool", 7, struct.pack("<?", True)),
        ("k.u64", 10, struct.pack("<Q", 1 << 40)),
        ("k.i64", 11, struct.pack("<q", -(1 << 40))),
        ("k.f64", 12, struct.pack("<d", 0.1)),
        ("k.arr_i32", 9, struct.pack("<IQ", 5, 3) + struct.pack("<3i", 1, -2, 3)),
        ("k.arr_str", 9, struct.pack("<IQ", 8, 2) + s_("ab") + s_("")),
    ]
    if alignment is not None:
        kvs.append(("general.alignment", 4, struct.pack("<I", alignment)))
    al = alignment or 32
    rng = np.random.default_rng(3)
    tensors = [  # name, ggml type, dims, data
        ("a.weight", 0, (3, 2), rng.standard_normal(6).astype(np.float32).tobytes()),
        ("b.weight", 2, (64, 2), rng.integers(0, 256, 2 * 2 * 18, dtype=np.uint8).tobytes()),
        ("c.weight", 14, (256, 1, 1), rng.integers(0, 256, 210, dtype=np.uint8).tobytes()),
    ]
    head = struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(kvs))
    for k, t, v in kvs:
        head += s_(k) + struct.pack("<I", t) + v
    offs, off = [], 0
    for name, ty, dims, data in tensors:
        head += s_(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        head += struct.pack("<IQ", ty, off)
        offs.append(off)
        off = (off + len(data) + al - 1) // al * al
    head += b"\0" * (-len(head) % al)
    body = bytearray(off)
    for (_, _, _, data), o in zip(tensors, offs):
        body[o:o + len(data)] = data
    return head + bytes(body), kvs, tensors


def spec_writer(alignment=None) -> G.GgufWriter:
    """The same content as spec_image, through the library's writer."""
    w = G.GgufWriter()
    w.kv("general.architecture", G.Value.String("qwen3"))
    w.kv("k.u8", G.Value(G.U8, 200))
    w.kv("k.i8", G.Value(G.I8, -5))
    w.kv("k.u16", G.Value(G.U16, 65000))
    w.kv("k.i16", G.Value(G.I16, -300))
    w.kv("k.u32", G.Value.U32(4000000000))
    w.kv("k.i32", G.Value.I32(-7))
    w.kv("adapter.lora.alpha", G.Value.F32(8.0))
    w.kv("k.bool", G.Value.Bool(True))
    w.kv("k.u64", G.Value.U64(1 << 40))
    w.kv("k.i64", G.Value.I64(-(1 << 40)))
    w.kv("k.f64", G.Value.F64(0.1))
    w.kv("k.arr_i32", G.Value.Array(G.I32, [1, -2, 3]))
    w.kv("k.arr_str", G.Value.Array(G.STRING, ["ab", ""]))
    if alignment is not None:
        w.kv("general.alignment", G.Value.U32(alignment))
    for name, ty, dims, data in spec_image(alignment)[2]:
        w.tensor(name, dims, ty, np.frombuffer(data, dtype=np.uint8))
    return w


@pytest.mark.parametrize("alignment", [None, 64, 4096])
def test_reader_decodes_spec_image(alignment):
    img, _, tensors = spec_image(alignment)
    g = G.GgufFile.from_bytes(img)
    assert g.version == 3
    assert g.get_str("general.architecture") == "qwen3"
    assert g.get("k.u8") == 200 and g.get("k.i8") == -5 and g.get("k.u16") == 65000 and g.get("k.i16") == -300
    assert g.get("k.u32") == 4000000000 and g.get("k.i32") == -7 and g.get("k.bool") is True
    assert g.get("k.u64") == 1 << 40 and g.get("k.i64") == -(1 << 40) and g.get("k.f64") == 0.1
    assert g.get_f32("adapter.lora.alpha") == 8.0  # src/rie.rs:379, tests/engine.rs:242
    assert g.get_f32("k.i32") == -7.0 and g.get_u32("k.u32") == 4000000000
    assert g.get_str("k.u32") is None and g.get_f32("general.architecture") is None
    assert g.get_str("missing") is None and g.get_f32("missing") is None and g.get("missing") is None
    assert list(g.get("k.arr_i32")) == [1, -2, 3] and g.get("k.arr_str") == ["ab", ""]
    assert len(g.tensors()) == 3 and g.tensor("nope") is None
    al = alignment or 32
    for (name, ty, dims, data), t in zip(tensors, g.tensors()):
        assert (t.name, t.ty, t.dims, t.nbytes) == (name, ty, dims, len(data))
        view = g.tensor_data(t)
        assert view.tobytes() == data
        assert (view.ctypes.data - g._keep[1].ctypes.data) % al == 0  # data start + offset aligned
    a = g.tensor("a.weight")
    assert (a.n_rows(), a.row_len()) == (2, 3)
    np.testing.assert_array_equal(g.tensor_f32(a), np.frombuffer(tensors[0][3], np.float32).reshape(2, 3))
    c = g.tensor("c.weight")
    assert (c.n_rows(), c.row_len()) == (1, 256)


@pytest.mark.parametrize("alignment", [None, 64, 4096])
def test_writer_reproduces_spec_image_bytes(alignment):
    img = spec_image(alignment)[0]
    w = spec_writer(alignment)
    assert w.to_bytes() == img
    assert w.to_bytes() == img  # the image is rebuilt on every call


def test_write_file_is_atomic_and_mapped_back(tmp_path):
    w = spec_writer(64)
    path = tmp_path / "m.gguf"
    w.write(path)
    assert not os.path.exists(str(path) + ".tmp")
    assert path.read_bytes() == w.to_bytes()
    with G.GgufFile.open(path) as g:
        assert g.get_str("general.architecture") == "qwen3"
        assert g.tensor_data(g.tensor("b.weight")).tobytes() == spec_image(64)[2][1][3]
    with pytest.raises(RtqError):
        G.GgufFile.open(tmp_path / "absent.gguf")
    with pytest.raises(RtqError):
        w.write(tmp_path / "no_such_dir" / "x.gguf")


def test_every_truncation_fails_cleanly():
    img, _, tensors = spec_image(64)
    end = len(img) - (-len(tensors[-1][3]) % 64)  # the last tensor's last byte; only padding follows
    for n in range(0, end):
        with pytest.raises(RtqError) as e:
            G.GgufFile.from_bytes(img[:n] if n else b"\0")
        assert e.value.status == 1
    # the padding after the last tensor carries nothing
    g = G.GgufFile.from_bytes(img[:end])
    assert g.tensor_data(g.tensor("c.weight")).tobytes() == tensors[-1][3]


def _patched(img: bytes, at: int, fmt: str, v) -> bytes:
    b = bytearray(img)
    struct.pack_into(fmt, b, at, v)
    return bytes(b)


def test_malformed_headers_are_rejected():
    img, _, tensors = spec_image()
    bad = [_patched(img, 0, "<I", 0x46554746),  # magic
           _patched(img, 4, "<I", 1),  # version 1
           _patched(img, 4, "<I", 4),  # version 4
           _patched(img, 8, "<Q", 1 << 30),  # tensor count
           _patched(img, 16, "<Q", 1000)]  # kv count beyond the image
    # first key's value type -> 13 (unknown)
    k0 = 24 + 8 + len("general.architecture")
    bad.append(_patched(img, k0, "<I", 13))
    # the array of i32 -> element type 9 (nested array)
    at = img.index(b"k.arr_i32") + len("k.arr_i32") + 4
    bad.append(_patched(img, at, "<I", 9))
    # a tensor's n_dims -> 5, its first dim -> 0, its offset unaligned, its offset past the end
    at = img.index(b"a.weight") + len("a.weight")
    bad += [_patched(img, at, "<I", 5), _patched(img, at + 4, "<Q", 0)]
    at = img.index(b"c.weight") + len("c.weight") + 4 + 3 * 8 + 4
    bad += [_patched(img, at, "<Q", 33), _patched(img, at, "<Q", 1 << 20)]
    for b in bad:
        with pytest.raises(RtqError):
            G.GgufFile.from_bytes(b)
    # alignment that is not a power of two, or not a u32
    w = G.GgufWriter()
    with pytest.raises(RtqError):
        w.kv("general.alignment", G.Value.U32(48))
    with pytest.raises(RtqError):
        w.kv("general.alignment", G.Value.U64(64))


def test_writer_checks_tensor_sizes():
    w = G.GgufWriter()
    with pytest.raises(RtqError):
        w.tensor("x", (64, 2), 2, np.zeros(2 * 2 * 18 - 1, np.uint8))  # one byte short
    with pytest.raises(RtqError):
        w.tensor("x", (100, 1), 12, np.zeros(144, np.uint8))  # 100 is not a whole Q4_K super-block
    with pytest.raises(RtqError):
        w.tensor("x", (4, 0), 0, np.zeros(0, np.uint8))  # zero dimension
    with pytest.raises(RtqError):
        w.tensor("x", (1, 1, 1, 1, 1), 0, np.zeros(4, np.uint8))  # five dims
    w.tensor("x", (4, 1), 0, np.zeros(16, np.uint8))
    assert len(G.GgufFile.from_bytes(w.to_bytes()).tensors()) == 1


@pytest.mark.parametrize("seed", range(4))
def test_round_trip_random_content(seed):
    rng = np.random.default_rng(seed)
    w = G.GgufWriter()
    al = int(2 ** rng.integers(0, 8))
    w.kv("general.alignment", G.Value.U32(al))
    expect_kv, expect_t = {}, []
    for i in range(int(rng.integers(0, 20))):
        kind = int(rng.integers(0, 4))
        key = f"key.{i}"
        if kind == 0:
            v = "".join(chr(int(c)) for c in rng.integers(32, 0x3000, int(rng.integers(0, 12))))
            w.kv(key, G.Value.String(v))
        elif kind == 1:
            v = float(np.float32(rng.standard_normal()))
            w.kv(key, G.Value.F32(v))
        elif kind == 2:
            v = rng.integers(-1000, 1000, int(rng.integers(0, 9))).astype(np.int64)
            w.kv(key, G.Value.Array(G.I64, v))
        else:
            v = [str(int(x)) for x in rng.integers(0, 1 << 30, int(rng.integers(0, 5)))]
            w.kv(key, G.Value.Array(G.STRING, v))
        expect_kv[key] = v
    for i in range(int(rng.integers(0, 12))):
        ty = int(rng.choice([0, 1, 2, 8, 12, 14]))
        be = G.GGML_BLOCK[ty][0]
        dims = (be * int(rng.integers(1, 4)),) + tuple(int(d) for d in rng.integers(1, 4, int(rng.integers(0, 4))))
        n = int(np.prod(dims))
        data = rng.integers(0, 256, G.ggml_nbytes(ty, n), dtype=np.uint8)
        w.tensor(f"t{i}", dims, ty, data)
        expect_t.append((f"t{i}", ty, dims, data))
    g = G.GgufFile.from_bytes(w.to_bytes())
    assert g.keys() == ["general.alignment"] + list(expect_kv)
    for k, v in expect_kv.items():
        got = g.get(k)
        if isinstance(v, np.ndarray):
            np.testing.assert_array_equal(got, v)
        else:
            assert got == v
    assert [(t.name, t.ty, t.dims) for t in g.tensors()] == [(n, t, d) for n, t, d, _ in expect_t]
    for t, (_, _, _, data) in zip(g.tensors(), expect_t):
        np.testing.assert_array_equal(g.tensor_data(t), data)


def test_synthetic_presets_match_the_benchmark_shapes():
    q = G.SyntheticSpec.preset("qwen3-0.6b", G.GGML_Q4_0)
    plan = q.plan()
    assert len(plan) == 1 + 28 * 11 + 1  # embed, 28 x (3 norms + 2 qk norms + 7 linears), output norm
    d = dict((n, (t, dims)) for n, t, dims in plan)
    assert d["token_embd.weight"] == (2, (1024, 151936)) and "output.weight" not in d  # tied
    assert d["blk.0.attn_q.weight"] == (2, (1024, 2048)) and d["blk.27.attn_k.weight"] == (2, (1024, 1024))
    assert d["blk.3.attn_output.weight"] == (2, (2048, 1024)) and d["blk.5.ffn_down.weight"] == (2, (3072, 1024))
    assert d["blk.0.ffn_gate.weight"] == (2, (1024, 3072)) and d["blk.0.attn_q_norm.weight"] == (0, (128,))
    # Q4_0 bytes: every linear + the embedding at 18 B per 32 weights, norms f32
    lin = 28 * (1024 * (2048 + 1024 + 1024 + 3 * 3072) + 2048 * 1024) + 151936 * 1024
    norms = 28 * (2 * 1024 + 2 * 128) + 1024
    assert sum(G.ggml_nbytes(t, int(np.prod(dims))) for _, t, dims in plan) == lin // 32 * 18 + 4 * norms
    k = dict((n, (t, dims)) for n, t, dims in G.SyntheticSpec.preset("qwen3-4b", G.GGML_Q4_K).plan())
    assert k["blk.0.attn_q.weight"] == (12, (2560, 4096)) and k["blk.0.ffn_up.weight"] == (12, (2560, 9728))
    assert k["blk.35.ffn_down.weight"] == (14, (9728, 2560)) and k["token_embd.weight"] == (14, (2560, 151936))
    ll = dict((n, (t, dims)) for n, t, dims in G.SyntheticSpec.preset("llama3-8b", G.GGML_Q8_0).plan())
    assert ll["output.weight"] == (8, (4096, 128256)) and ll["blk.31.ffn_down.weight"] == (8, (14336, 4096))
    assert "blk.0.attn_q_norm.weight" not in ll
    assert G.SyntheticSpec.preset("nope", 2) is None


@pytest.mark.parametrize("wtype", [2, 8, 12, 14, 0])
def test_synthetic_tiny_build_contents(wtype):
    s = G.SyntheticSpec.tiny("qwen3", wtype)
    s.n_layer = 1
    s.tied_output = False
    g = G.GgufFile.from_bytes(s.build())
    a = s.arch
    assert g.get_str("general.architecture") == "qwen3"
    for key, v in [("block_count", 1), ("embedding_length", 256), ("feed_forward_length", 512),
                   ("attention.head_count", 4), ("attention.head_count_kv", 2), ("attention.key_length", 64),
                   ("rope.dimension_count", 64), ("vocab_size", 512)]:
        assert g.get_u32(f"{a}.{key}") == v, key
    assert g.get_f32(f"{a}.rope.freq_base") == 1e6
    plan = s.plan()
    assert [t.name for t in g.tensors()] == [n for n, _, _ in plan]
    for i, (name, ty, dims) in enumerate(plan):
        t = g.tensor(name)
        assert (t.ty, t.dims) == (ty, dims)
        raw = g.tensor_data(t)
        if name.endswith("norm.weight"):
            np.testing.assert_array_equal(raw.view(np.float32), 1.0)
            continue
        w = Rng(s.seed * 1_000_003 + i).vec_normal(int(np.prod(dims)), 0.02).reshape(-1, dims[0])
        want = w.view(np.uint8).reshape(-1) if ty == 0 else QUANTIZERS[ty](w).reshape(-1)
        np.testing.assert_array_equal(raw, want, err_msg=name)


def test_adapter_gguf_layout_round_trips():
    """The llama.cpp LoRA GGUF of write_gguf_adapter (src/rie.rs:349-363): lora_a has dims
    [in, rank] (rank rows of length in), lora_b [rank, out]; read back as read_gguf_adapter does
    (src/rie.rs:370-384)."""
    rng = Rng(5)
    r, inp, out = 4, 64, 96
    A = rng.vec_normal(r * inp, 0.1)
    B = rng.vec_normal(out * r, 0.1)
    w = G.GgufWriter()
    w.kv("general.architecture", G.Value.String("qwen3"))
    w.kv("general.type", G.Value.String("adapter"))
    w.kv("adapter.type", G.Value.String("lora"))
    w.kv("adapter.lora.alpha", G.Value.F32(8.0))
    w.tensor("blk.0.attn_q.weight.lora_a", [inp, r], 0, A)
    w.tensor("blk.0.attn_q.weight.lora_b", [r, out], 0, B)
    g = G.GgufFile.from_bytes(w.to_bytes())
    assert g.get_str("general.type") == "adapter" and g.get_str("adapter.type") == "lora"
    assert g.get_f32("adapter.lora.alpha") == 8.0
    ta, tb = g.tensor("blk.0.attn_q.weight.lora_a"), g.tensor("blk.0.attn_q.weight.lora_b")
    assert (ta.n_rows(), ta.row_len(), tb.n_rows(), tb.row_len()) == (r, inp, out, r)
    np.testing.assert_array_equal(g.tensor_f32(ta).reshape(-1), A)
    np.testing.assert_array_equal(g.tensor_f32(tb).reshape(-1), B)
