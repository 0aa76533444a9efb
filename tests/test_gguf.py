"""CPU tests of the GGUF v3 tensor reader (tc_gguf_* in libtc_hip.so; no GPU
call). Files come from tests/gguf_write.py (this build's writer, from the
published format). Where the compiled reference (oracle/_ref) exists, the
reference's own GGUFLoader reads the same files and every record, tensor byte
and parsed config value must agree; the format's own invariants (data offset,
alignment, byte sizes) and malformed-file refusals are checked either way."""
import os

import numpy as np
import pytest

import gguf_write as W
import oracle as O

Q8_0, Q4_K, Q5_K, Q6_K, IQ3_XXS, F32, F16 = 8, 12, 13, 14, 18, 0, 1


@pytest.fixture(scope="module")
def lib():
    import tc_hip
    return tc_hip.load_library()


@pytest.fixture(scope="module")
def ref():
    if not O.available_reference():
        pytest.skip("compiled reference (oracle/_ref) not built here")
    return O.Reference()


def loader(lib):
    import tc_hip
    return tc_hip.GGUFLoader(lib)


def qwen2_metadata():
    """Keys the reference's config parser reads, plus one of every value type."""
    return [
        ("general.architecture", W.STRING, "qwen2"),
        ("general.name", W.STRING, "synthetic qwen2 – test"),
        ("qwen2.block_count", W.U32, 28),
        ("qwen2.context_length", W.U32, 32768),
        ("qwen2.embedding_length", W.U32, 3584),
        ("qwen2.feed_forward_length", W.U32, 18944),
        ("qwen2.attention.head_count", W.U32, 28),
        ("qwen2.attention.head_count_kv", W.ARRAY, (W.U32, [4] * 28)),  # per-layer array: first element
        ("qwen2.rope.freq_base", W.F32, 1000000.0),
        ("qwen2.vocab_size", W.U64, 152064),
        ("qwen2.rope.dimension_sections", W.ARRAY, (W.I32, [11, 11, 10, 0])),
        ("qwen2.final_logit_softcapping", W.F64, 30.5),
        ("qwen2.expert_count", W.I32, 128),
        ("qwen2.expert_used_count", W.U16, 8),
        ("qwen2.expert_feed_forward_length", W.I64, 768),
        ("qwen2.rope.dimension_count", W.U8, 128),
        ("t.i8", W.I8, -5),
        ("t.i16", W.I16, -300),
        ("t.bool", W.BOOL, 1),
        ("t.boolf", W.BOOL, 0),
        ("t.f32", W.F32, 0.1),
        ("t.strarr", W.ARRAY, (W.STRING, ["a", "bb", ""])),
        ("t.emptyarr", W.ARRAY, (W.F32, [])),
        ("t.f64arr", W.ARRAY, (W.F64, [2.5, 3.5])),
        ("prism.hadamard.sign_widths", W.ARRAY, (W.I32, [1, 2, 3])),
        ("tokenizer.ggml.tokens", W.ARRAY, (W.STRING, ["<s>", "</s>", "x" * 70])),
    ]


def model_tensors(rng):
    def blocks(t, rows, cols):
        from qdata import random_blocks
        return random_blocks(t, rng, rows, cols)
    return [
        ("token_embd.weight", Q6_K, (512, 40), blocks(Q6_K, 40, 512)),
        ("blk.0.attn_q.weight", Q4_K, (512, 64), blocks(Q4_K, 64, 512)),
        ("blk.0.attn_k.weight", Q5_K, (256, 16), blocks(Q5_K, 16, 256)),
        ("blk.0.attn_v.weight", Q8_0, (512, 8), blocks(Q8_0, 8, 512)),
        ("blk.0.ffn_gate.weight", IQ3_XXS, (768, 24), blocks(IQ3_XXS, 24, 768)),
        ("blk.0.attn_norm.weight", F32, (512,), rng.integers(0, 256, 2048, dtype=np.uint8)),
        ("blk.0.ffn_gate_exps.weight", Q4_K, (256, 32, 4), blocks(Q4_K, 128, 256)),
        ("output_norm.weight", F16, (37,), rng.integers(0, 256, 74, dtype=np.uint8)),
    ]


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    rng = np.random.default_rng(2024)
    tensors = model_tensors(rng)
    path = str(tmp_path_factory.mktemp("gguf") / "model.gguf")
    W.write_gguf(path, qwen2_metadata(), tensors)
    return path, tensors


def test_records_bytes_and_layout(lib, model_file):
    path, tensors = model_file
    g = loader(lib)
    assert g.load(path), g.last_error
    assert g.version == 3
    recs = g.tensorRecords()
    assert [r.name for r in recs] == [t[0] for t in tensors]
    raw = open(path, "rb").read()
    assert g.data_offset % 32 == 0
    for r, (name, t, dims, data) in zip(recs, tensors):
        assert r.type == t and r.shape == tuple(dims)
        assert r.bytes == len(data)  # blocks x block bytes
        assert r.offset % 32 == 0
        got = g.getTensor(name)
        assert np.array_equal(got, np.asarray(data, np.uint8))
        start = g.data_offset + r.offset
        assert raw[start:start + r.bytes] == got.tobytes()
        assert g.getTensorInfo(name).index == r.index
    assert g.getTensorInfo("missing") is None and g.getTensor("missing") is None
    g.close()


def test_metadata_rendering(lib, model_file):
    g = loader(lib)
    assert g.load(model_file[0])
    m = g.metadata
    assert m("general.architecture") == "qwen2"
    assert m("general.name") == "synthetic qwen2 – test"
    assert m("qwen2.block_count") == "28"
    assert m("qwen2.attention.head_count_kv") == "4"
    assert m("qwen2.rope.freq_base") == "1000000.000000"
    assert m("qwen2.vocab_size") == "152064"
    assert m("qwen2.rope.dimension_sections") == "11,11,10,0"
    assert m("qwen2.final_logit_softcapping") == "30.500000"
    assert m("t.i8") == "-5" and m("t.i16") == "-300"
    assert m("t.bool") == "true" and m("t.boolf") == "false"
    assert m("t.f32") == "0.100000"
    assert m("t.f64arr") == "2.500000"
    for absent in ("t.strarr", "t.emptyarr", "prism.hadamard.sign_widths", "tokenizer.ggml.tokens", "nope"):
        assert m(absent) is None, absent
    g.close()


def test_matches_compiled_reference_loader(lib, ref, model_file):
    path, tensors = model_file
    r = O.RefGGUF(ref, path)
    assert r.ok
    g = loader(lib)
    assert g.load(path)
    ours = g.tensorRecords()
    theirs = r.records()
    assert len(ours) == len(theirs)
    for a, (name, t, dims, off) in zip(ours, theirs):
        assert (a.name, a.type, a.shape, a.offset) == (name, t, dims, off)
        assert np.array_equal(g.getTensor(a.name), r.tensor(a.name, a.bytes))
    c = r.config()
    m = g.metadata
    assert c["architecture"] == m("general.architecture") and c["modelName"] == m("general.name")
    for key, field in [("block_count", "numLayers"), ("context_length", "maxSeqLen"),
                       ("embedding_length", "hiddenSize"), ("feed_forward_length", "intermediateSize"),
                       ("attention.head_count", "numAttentionHeads"), ("attention.head_count_kv", "numKVHeads"),
                       ("vocab_size", "vocabSize"), ("expert_count", "expertCount"),
                       ("expert_used_count", "expertUsedCount"),
                       ("expert_feed_forward_length", "expertFeedForwardLength"),
                       ("rope.dimension_count", "ropeDimensionCount")]:
        assert int(m("qwen2." + key)) == c[field], key
    assert [int(v) for v in m("qwen2.rope.dimension_sections").split(",")] == [c[f"sec{i}"] for i in range(4)]
    assert np.float32(float(m("qwen2.rope.freq_base"))) == np.float32(c["ropeTheta"])
    assert np.float32(float(m("qwen2.final_logit_softcapping"))) == np.float32(c["finalLogitSoftcapping"])
    r.close()
    rm = O.RefGGUF(ref, path, metadata_only=True)
    gm = loader(lib)
    assert rm.ok and gm.loadMetadata(path)
    assert [(a.name, a.type, a.shape, a.offset) for a in gm.tensorRecords()] == rm.records()
    assert gm.getTensor("blk.0.attn_q.weight") is None  # metadata only: no data
    rm.close()


def test_block_geometry_matches_reference(lib, ref):
    for t in list(range(0, 32)) + [200]:
        assert lib.tc_gguf_block_size(t) == ref.lib.ref_ggml_block_size(t), t
        if t == 19:
            continue  # IQ1_S: GGML's block is 50 bytes (the reference's table says 34)
        assert lib.tc_gguf_type_size(t) == ref.lib.ref_ggml_type_size(t), t


def test_general_alignment_key(lib, tmp_path):
    rng = np.random.default_rng(3)
    tensors = [("a", Q4_K, (256, 3), rng.integers(0, 256, 432, dtype=np.uint8)),
               ("b", F32, (5,), rng.integers(0, 256, 20, dtype=np.uint8)),
               ("c", Q8_0, (64, 2), rng.integers(0, 256, 136, dtype=np.uint8))]
    path = str(tmp_path / "a64.gguf")
    W.write_gguf(path, [("general.architecture", W.STRING, "x")], tensors, alignment=64, set_alignment_key=True)
    g = loader(lib)
    assert g.load(path), g.last_error
    assert g.data_offset % 64 == 0
    for name, _, _, data in tensors:
        assert np.array_equal(g.getTensor(name), data)
    g.close()


def test_malformed_files_are_refused(lib, tmp_path, model_file):
    import struct
    path, _ = model_file
    raw = open(path, "rb").read()
    g = loader(lib)
    bad = tmp_path / "bad.gguf"

    def refused(data):
        bad.write_bytes(data)
        ok = g.load(str(bad))
        g.close()
        return not ok

    assert refused(b"GGUF")  # too short
    assert refused(b"GGUG" + raw[4:])  # magic
    assert refused(raw[:4] + struct.pack("<I", 2) + raw[8:])  # version 2
    assert refused(raw[:8] + struct.pack("<Q", 1 << 60) + raw[16:])  # tensor count
    # every truncation inside the header, metadata and records, and of the data
    cut_points = sorted(set(list(range(0, 600, 7)) + list(range(600, len(raw) - 1, 997)) + [len(raw) - 1]))
    for n in cut_points:  # the last tensor ends at the end of the file
        assert refused(raw[:n]), n
    assert g.last_error.startswith("gguf:")
    assert not g.load(str(tmp_path / "does_not_exist.gguf"))
    assert "cannot open" in g.last_error


def test_dimension_limit(lib, tmp_path):
    path = str(tmp_path / "d5.gguf")
    W.write_gguf(path, [], [("t", F32, (1, 1, 1, 1, 2), np.zeros(8, np.uint8))])
    g = loader(lib)
    assert not g.load(path)
    assert "dimensions" in g.last_error
