"""The GGUF reader (bb_gguf_*), on the CPU: the reference's own parser, config and tensor tests
re-created on the same hand-built bytes (gguf.rs:431-659, config.rs:108-240, tensor.rs:135-167,
model.rs:709-727), the tensor-table check, a synthetic model's round trip through the writer,
and malformed input (every truncation and random corruption of a valid file returns an error
code or parses; nothing crashes)."""
import struct

import numpy as np
import pytest

from bebelm_amd import _lib, gguf, synth
from bebelm_amd._lib import BBError

VT_U8, VT_I16, VT_U32, VT_F32, VT_STRING, VT_ARRAY, VT_I64, VT_F64 = 0, 3, 4, 6, 8, 9, 11, 12


def push_str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def build_sample():
    """gguf.rs:441-490: version 3, two F32 tensors, three metadata keys, 32-byte alignment."""
    b = b"GGUF" + struct.pack("<IQQ", 3, 2, 3)
    b += push_str("general.architecture") + struct.pack("<I", VT_STRING) + push_str("lfm2_moe")
    b += push_str("lfm2_moe.block_count") + struct.pack("<II", VT_U32, 24)
    b += push_str("tokenizer.ggml.tokens") + struct.pack("<IIQ", VT_ARRAY, VT_STRING, 2)
    b += push_str("<bos>") + push_str("hello")
    b += push_str("a") + struct.pack("<IQIQ", 1, 4, 0, 0)
    b += push_str("b") + struct.pack("<IQQIQ", 2, 2, 3, 0, 16)
    b += b"\0" * (-len(b) % 32)
    b += struct.pack("<4f", 1, 2, 3, 4) + struct.pack("<6f", 10, 11, 12, 13, 14, 15)
    return b


def header(tensor_count, kv_count, body):
    """gguf.rs:543-553."""
    b = b"GGUF" + struct.pack("<IQQ", 3, tensor_count, kv_count) + body
    return b + b"\0" * (-len(b) % 32)


def parse_err(data):
    with pytest.raises(BBError) as e:
        gguf.GgufFile.from_bytes(data)
    return e.value


# ---- gguf.rs tests ------------------------------------------------------------------------------

def test_parses_header_and_metadata():
    g = gguf.GgufFile.from_bytes(build_sample())
    assert (g.version, g.alignment) == (3, 32)
    assert g.architecture() == "lfm2_moe"
    assert g.get_u32("lfm2_moe.block_count") == 24
    assert g.meta_type("tokenizer.ggml.tokens") == (VT_ARRAY, VT_STRING, 2)
    assert g.get_str_array("tokenizer.ggml.tokens") == ["<bos>", "hello"]
    assert g.keys == ["general.architecture", "lfm2_moe.block_count", "tokenizer.ggml.tokens"]


def test_parses_tensors_and_data():
    g = gguf.GgufFile.from_bytes(build_sample())
    a, b = g.tensors
    assert (a.name, a.dims, a.ggml_type, a.n_elements(), a.data_len) == ("a", [4], 0, 4, 16)
    assert (b.name, b.dims, b.n_elements()) == ("b", [2, 3], 6)
    assert g.tensor_data(a).view(np.float32).tolist() == [1.0, 2.0, 3.0, 4.0]
    assert g.tensor_data(b).view(np.float32)[0] == 10.0
    assert g.data_offset % 32 == 0 and b.data_start == g.data_offset + 16


def test_rejects_bad_magic():
    d = bytearray(build_sample())
    d[0] = ord("X")
    e = parse_err(bytes(d))
    assert e.code == _lib.BB_ERR_FORMAT and "not a GGUF file (magic = [88, 71, 85, 70])" in str(e)


def test_rejects_truncated_file():
    e = parse_err(build_sample()[:10])
    assert e.code == _lib.BB_ERR_FORMAT and "unexpected end of file: need 8 bytes at offset 8, file is 10 bytes" in str(e)


def test_rejects_unsupported_version():
    d = bytearray(build_sample())
    d[4:8] = struct.pack("<I", 5)
    assert "unsupported GGUF version 5" in str(parse_err(bytes(d)))


def test_rejects_unknown_value_type():
    body = push_str("weird") + struct.pack("<I", 99)
    assert "unknown metadata value type 99" in str(parse_err(header(0, 1, body)))


def test_rejects_unknown_tensor_type():
    body = push_str("weird") + struct.pack("<IQIQ", 1, 1, 1000, 0)
    assert "tensor 'weird' has unmodeled ggml type 1000" in str(parse_err(header(1, 0, body)))


def test_rejects_tensor_out_of_bounds():
    body = push_str("big") + struct.pack("<IQIQ", 1, 1024, 0, 0)
    assert "tensor 'big' data range falls outside the file" in str(parse_err(header(1, 0, body)))


def test_reads_custom_alignment():
    body = push_str("general.alignment") + struct.pack("<II", VT_U32, 8)
    assert gguf.GgufFile.from_bytes(header(0, 1, body)).alignment == 8


def test_accessors_widen_integer_and_float_types():
    body = push_str("k.u8") + struct.pack("<IB", VT_U8, 7)
    body += push_str("k.i64") + struct.pack("<Iq", VT_I64, 123)
    body += push_str("k.f64") + struct.pack("<Id", VT_F64, 2.5)
    body += push_str("k.i16arr") + struct.pack("<IIQ3h", VT_ARRAY, VT_I16, 3, 10, 0, 8)
    g = gguf.GgufFile.from_bytes(header(0, 4, body))
    assert g.get_u32("k.u8") == 7 and g.get_u32("k.i64") == 123
    assert g.get_f32("k.f64") == 2.5
    assert g.get_u32_array("k.i16arr") == [10, 0, 8]


# ---- beyond the reference's tests: Rust's conversions and None results -------------------------

def test_accessor_conversions_follow_rust_as_casts():
    body = push_str("neg8") + struct.pack("<Ib", 1, -1)            # I8 -1 as u32 = 0xFFFFFFFF
    body += push_str("big64") + struct.pack("<IQ", 10, (1 << 40) + 5)  # U64 truncates to its low 32 bits
    body += push_str("f") + struct.pack("<If", VT_F32, 0.1)
    body += push_str("s") + struct.pack("<I", VT_STRING) + push_str("x")
    body += push_str("mixed") + struct.pack("<IIQ", VT_ARRAY, VT_STRING, 1) + push_str("a")
    body += push_str("flag") + struct.pack("<IB", 7, 1)
    g = gguf.GgufFile.from_bytes(header(0, 6, body))
    assert g.get_u32("neg8") == 0xFFFFFFFF and g.get_u32("big64") == 5
    assert g.get_f32("f") == np.float32(0.1)
    assert g.get_u32("s") is None and g.get_f32("s") is None and g.get_str("f") is None
    assert g.get_u32_array("mixed") is None and g.get_u32_array("s") is None
    assert g.get_u32("flag") is None            # Bool is not an integer for get_u32
    assert g.get_u32("absent") is None and g.tensor("absent") is None


def test_nested_arrays_and_repeated_keys():
    inner = struct.pack("<IQ", VT_U32, 2) + struct.pack("<2I", 1, 2)
    body = push_str("nest") + struct.pack("<IIQ", VT_ARRAY, VT_ARRAY, 2) + inner + inner
    body += push_str("k") + struct.pack("<II", VT_U32, 1) + push_str("k") + struct.pack("<II", VT_U32, 2)
    g = gguf.GgufFile.from_bytes(header(0, 3, body))
    assert g.meta_type("nest") == (VT_ARRAY, VT_ARRAY, 2)
    assert g.get_u32("k") == 2 and g.keys == ["nest", "k"]   # HashMap::insert keeps the last value


def test_invalid_utf8_is_rejected():
    body = struct.pack("<Q", 2) + b"\xc3\x28" + struct.pack("<II", VT_U32, 1)
    assert "invalid UTF-8 in a GGUF string" in str(parse_err(header(0, 1, body)))
    ok = push_str("café€\U0001F600") + struct.pack("<II", VT_U32, 1)
    assert gguf.GgufFile.from_bytes(header(0, 1, ok)).get_u32("café€\U0001F600") == 1
    for bad in (b"\xc0\x80", b"\xed\xa0\x80", b"\xf4\x90\x80\x80", b"\xe2\x82"):  # overlong, surrogate, > U+10FFFF, cut
        body = struct.pack("<Q", len(bad)) + bad + struct.pack("<II", VT_U32, 1)
        parse_err(header(0, 1, body))


def test_open_maps_a_file_and_reports_io_errors(tmp_path):
    p = tmp_path / "s.gguf"
    p.write_bytes(build_sample())
    with gguf.GgufFile.open(p) as g:
        assert [t.name for t in g.tensors] == ["a", "b"]
        assert g.tensor_data(g.tensors[0]).view(np.float32).tolist() == [1.0, 2.0, 3.0, 4.0]
    with pytest.raises(BBError) as e:
        gguf.GgufFile.open(tmp_path / "absent.gguf")
    assert e.value.code == _lib.BB_ERR_IO and "io error: No such file or directory (os error 2)" in str(e.value)
    (tmp_path / "empty.gguf").write_bytes(b"")
    with pytest.raises(BBError) as e:
        gguf.GgufFile.open(tmp_path / "empty.gguf")
    assert e.value.code == _lib.BB_ERR_FORMAT


def test_tensor_views_outlive_the_file_object(tmp_path):
    # a zero-copy view holds the mapping: after close(), and after the GgufFile is collected, it
    # still reads the tensor's bytes; the mapping goes with the last view
    import gc
    import weakref

    p = tmp_path / "s.gguf"
    p.write_bytes(build_sample())
    g = gguf.GgufFile.open(p)
    a = g.tensor_data(g.tensors[0])
    g.close()
    assert g.handle is None
    with pytest.raises(BBError):
        g.tensor_data(g.tensors[0])
    assert a.view(np.float32).tolist() == [1.0, 2.0, 3.0, 4.0]
    b = gguf.GgufFile.open(p).tensor_data(gguf.GgufFile.open(p).tensors[1])
    gc.collect()
    assert b.view(np.float32).tolist() == [10.0, 11.0, 12.0, 13.0, 14.0, 15.0]
    g2 = gguf.GgufFile.from_bytes(build_sample())
    owner = weakref.ref(g2._map)
    c = g2.tensor_data(g2.tensors[1])[:8]
    del g2
    gc.collect()
    assert owner() is not None and c.view(np.float32).tolist() == [10.0, 11.0]
    del a, b, c
    gc.collect()
    assert owner() is None


# ---- tensor.rs:135-167: block sizes and byte sizes, through the table ---------------------------

@pytest.mark.parametrize("ty,n,nbytes", [(12, 2048 * 2048, 2_359_296), (14, 256, 210), (8, 32, 34), (0, 10, 40),
                                         (1, 3, 6), (30, 3, 6), (28, 2, 16), (15, 256, 292), (2, 64, 36)])
def test_byte_size_math(ty, n, nbytes):
    body = push_str("t") + struct.pack("<IQIQ", 1, n, ty, 0)
    g = gguf.GgufFile.from_bytes(header(1, 0, body) + b"\0" * nbytes)
    assert g.tensors[0].data_len == nbytes


@pytest.mark.parametrize("ty,n", [(12, 100), (99, 4), (4, 1), (29, 1)])
def test_unmodelled_type_or_partial_block_is_rejected(ty, n):
    body = push_str("t") + struct.pack("<IQIQ", 1, n, ty, 0)
    assert "has unmodeled ggml type" in str(parse_err(header(1, 0, body) + b"\0" * 4096))


# ---- config.rs:108-240 ---------------------------------------------------------------------------

SCHEDULE = [8 if i in synth.ATTENTION_LAYERS else 0 for i in range(24)]


def build_config_gguf(arch="lfm2moe", block_count=24, schedule=SCHEDULE, overrides=None):
    """config.rs:154-188: tensor-free, metadata matching the constants except the knobs varied."""
    u32s = {"block_count": block_count, "embedding_length": 2048, "vocab_size": 128000,
            "attention.head_count": 32, "expert_count": 32, "expert_used_count": 4, "feed_forward_length": 7168,
            "expert_feed_forward_length": 1792, "leading_dense_block_count": 2, "shortconv.l_cache": 3}
    f32s = {"rope.freq_base": 5_000_000.0, "attention.layer_norm_rms_epsilon": 1e-5}
    for k, v in (overrides or {}).items():
        (u32s if k in u32s else f32s)[k] = v
    kvs = b"".join(push_str("lfm2moe." + k) + struct.pack("<II", VT_U32, v) for k, v in u32s.items())
    kvs += push_str("general.architecture") + struct.pack("<I", VT_STRING) + push_str(arch)
    kvs += b"".join(push_str("lfm2moe." + k) + struct.pack("<If", VT_F32, v) for k, v in f32s.items())
    kvs += push_str("lfm2moe.attention.head_count_kv") + struct.pack("<IIQ", VT_ARRAY, VT_U32, len(schedule))
    kvs += struct.pack(f"<{len(schedule)}I", *schedule)
    return header(0, len(u32s) + len(f32s) + 2, kvs)


def validate_err(data):
    g = gguf.GgufFile.from_bytes(data)
    with pytest.raises(BBError) as e:
        g.validate()
    return e.value


def test_validate_accepts_matching_metadata():
    gguf.GgufFile.from_bytes(build_config_gguf()).validate()


def test_validate_rejects_wrong_architecture():
    assert 'architecture: expected "lfm2moe", got "llama"' in str(validate_err(build_config_gguf(arch="llama")))


def test_validate_rejects_wrong_block_count():
    assert "lfm2moe.block_count: expected 24, got 12" in str(validate_err(build_config_gguf(block_count=12)))


def test_validate_rejects_schedule_mismatch():
    e = validate_err(build_config_gguf(schedule=[0] * 24))
    assert "layer 2: head_count_kv=0, expected 8 (schedule mismatch)" in str(e)
    assert "head_count_kv has 23 entries, expected 24" in str(validate_err(build_config_gguf(schedule=SCHEDULE[:23])))


def test_validate_float_tolerances_and_missing_keys():
    gguf.GgufFile.from_bytes(build_config_gguf(overrides={"rope.freq_base": 5_000_000.5})).validate()
    e = validate_err(build_config_gguf(overrides={"rope.freq_base": 5_000_002.0}))
    assert "lfm2moe.rope.freq_base: expected 5000000, got 5000002" in str(e)
    e = validate_err(build_config_gguf(overrides={"attention.layer_norm_rms_epsilon": 1e-6}))
    assert "lfm2moe.attention.layer_norm_rms_epsilon: expected 0.00001, got 0.000001" in str(e)
    e = validate_err(header(0, 1, push_str("general.architecture") + struct.pack("<I", VT_STRING) + push_str("lfm2moe")))
    assert e.code == _lib.BB_ERR_MISSING and "missing metadata lfm2moe.block_count" in str(e)
    assert validate_err(header(0, 0, b"")).code == _lib.BB_ERR_MISSING


# ---- model.rs:572-584, :619-660, :709-727: the tensor table --------------------------------------

def small_full_schedule():
    """The real 24-layer schedule (attention on 2, 6, 10, 14, 18, 21; dense FFN on 0 and 1) at
    small sizes, so the file is a few MB."""
    return synth.model_weights(seed=3, hidden=256, vocab=300, moe_ff=256, dense_ff=512, n_experts=4, n_heads=4,
                               n_kv_heads=2)


def test_expected_tensor_count_matches_file():
    mw = small_full_schedule()
    g = gguf.GgufFile.from_bytes(synth.model_gguf(mw).to_bytes())
    assert g.check_tensors() == 256 == len(g.tensors)                 # model.rs:709-713
    assert len({t.name for t in g.tensors}) == 256                    # model.rs:715-727


def test_check_tensors_reports_missing_and_misshaped():
    mw = small_full_schedule()
    w = synth.model_gguf(mw)
    w.tensors = [t for t in w.tensors if t[0] != "blk.3.ffn_norm.weight"]
    g = gguf.GgufFile.from_bytes(w.to_bytes())
    with pytest.raises(BBError) as e:
        g.check_tensors()
    assert e.value.code == _lib.BB_ERR_MISSING and "missing tensor blk.3.ffn_norm.weight" in str(e.value)
    w = synth.model_gguf(mw)
    i = [t[0] for t in w.tensors].index("blk.2.attn_k.weight")
    name, dims, ty, data = w.tensors[i]
    w.tensors[i] = (name, [256, 64], ty, data[: len(data) // 2])
    g = gguf.GgufFile.from_bytes(w.to_bytes())
    with pytest.raises(BBError) as e:
        g.check_tensors()
    assert "tensor blk.2.attn_k.weight: shape [256, 64] != expected [256, 128]" in str(e.value)


def test_synthetic_model_round_trips_through_the_writer(tmp_path):
    mw = synth.model_weights(seed=5, hidden=512, vocab=1000, n_layers=6, n_dense=1, attention_layers=(1, 4),
                             moe_ff=512, dense_ff=1024, n_experts=8, n_heads=8, n_kv_heads=2)
    w = synth.model_gguf(mw)
    path = tmp_path / "m.gguf"
    w.save(path)
    with gguf.GgufFile.open(path) as g:
        assert g.check_tensors() == len(g.tensors) == len(w.tensors)
        for name, dims, ty, data in w.tensors:
            t = g.tensor(name)
            assert (t.dims, t.ggml_type) == (dims, ty)
            assert t.data_start % 32 == 0
            assert np.array_equal(g.tensor_data(t), np.frombuffer(data, np.uint8)), name
        assert g.get_u32_array("lfm2moe.attention.head_count_kv") == [0, 2, 0, 0, 2, 0]
        assert g.get_u32("lfm2moe.leading_dense_block_count") == 1
        assert g.get_f32("lfm2moe.attention.layer_norm_rms_epsilon") == np.float32(1e-5)
        with pytest.raises(BBError):
            g.validate()                                               # not LFM2.5-8B-A1B's sizes


# ---- malformed input -------------------------------------------------------------------------------

def small_file():
    mw = synth.model_weights(seed=7, hidden=256, vocab=40, n_layers=3, n_dense=1, attention_layers=(1,), moe_ff=256,
                             dense_ff=256, n_experts=2, n_heads=4, n_kv_heads=2)
    return synth.model_gguf(mw).to_bytes()


def test_every_truncation_is_an_error():
    data = small_file()
    g = gguf.GgufFile.from_bytes(data)
    head = g.data_offset
    for n in list(range(0, head + 64)) + list(range(head + 64, len(data), 997)):
        with pytest.raises(BBError) as e:
            gguf.GgufFile.from_bytes(data[:n])
        assert e.value.code == _lib.BB_ERR_FORMAT, n
    gguf.GgufFile.from_bytes(data)


def test_random_corruption_never_crashes():
    data = small_file()
    head = gguf.GgufFile.from_bytes(data).data_offset
    rng = np.random.default_rng(11)
    outcomes = set()
    for trial in range(3000):
        d = bytearray(data)
        for _ in range(int(rng.integers(1, 4))):
            d[int(rng.integers(0, head))] = int(rng.integers(0, 256))
        try:
            g = gguf.GgufFile.from_bytes(bytes(d))
            for t in g.tensors:
                assert t.data_start + t.data_len <= len(d)
            outcomes.add("ok")
        except BBError as e:
            assert e.code in (_lib.BB_ERR_FORMAT, _lib.BB_ERR_OOM), e
            outcomes.add(e.code)
    assert "ok" in outcomes and _lib.BB_ERR_FORMAT in outcomes
