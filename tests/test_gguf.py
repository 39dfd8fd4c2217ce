"""GGUF v3 reader (af_gguf_*, the C ABI's GgufInspector) on the reference's own fixtures
(crates/model-formats/src/gguf.rs:546-662) and on a synthetic Gemma 4 file written byte for byte
(tests/gguf_writer.py).  Host code only: these run without a GPU."""
import os

import numpy as np
import pytest

from adaforge_amd import synth
from adaforge_amd._native import AfError
from adaforge_amd.gguf import ArraySummary, GgufFile, GgufInspector
from tests import gguf_writer as W


def write(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def test_reads_quantized_tensor_and_rejects_truncation_gguf_rs_597(tmp_path):
    b = W.reference_fixture()
    m = GgufInspector().inspect(write(tmp_path, "a.gguf", b))
    assert m.format_version == 3 and m.data_offset == 64 and m.file_bytes == len(b)
    (t,) = m.tensors
    assert t.name == "x" and t.dimensions == [32] and t.weight_type == "Q4_0" and t.byte_length == 18
    assert t.file_offset == 64
    for n in range(len(b)):
        with pytest.raises(AfError):
            GgufInspector().inspect(write(tmp_path, f"t{n}.gguf", b[:n]))


@pytest.mark.parametrize("pos,value", [(0, 0), (4, 2), (45, 99), (49, 1)])
def test_rejects_bad_signature_version_type_and_offset_gguf_rs_608(tmp_path, pos, value):
    b = bytearray(W.reference_fixture())
    b[pos] = value
    with pytest.raises(AfError):
        GgufInspector().inspect(write(tmp_path, "bad.gguf", bytes(b)))


def test_preserves_array_values_and_q6k_layout_gguf_rs_635(tmp_path):
    m = GgufInspector().inspect(write(tmp_path, "m.gguf", W.reference_model(224, 32)))
    assert m.tensors[0].byte_length == 210 and m.tensors[1].byte_length == 210
    assert m.metadata["gemma4.test"] == [True, False]
    assert m.metadata["general.alignment"] == 32


@pytest.mark.parametrize("offset,alignment", [(0, 32), (1, 32), (224, 0), (224, 3)])
def test_rejects_overlaps_unaligned_offsets_and_invalid_alignment_gguf_rs_644(tmp_path, offset, alignment):
    with pytest.raises(AfError):
        GgufInspector().inspect(write(tmp_path, "m.gguf", W.reference_model(offset, alignment)))


def test_rejects_duplicates_unknown_types_and_zero_dimensions(tmp_path):
    q4 = bytes(18)
    cases = {
        "duplicate key": ([("k", W.U32, 1), ("k", W.U32, 2)], [("t", W.T_Q4_0, [32], q4)]),
        "duplicate tensor": ([], [("t", W.T_Q4_0, [32], q4), ("t", W.T_Q4_0, [32], q4)]),
        "zero dimension": ([], [("t", W.T_F32, [0], b"")]),
        "partial block": ([], [("t", W.T_Q4_0, [16], bytes(18))]),
        "nested array": ([("k", W.ARRAY, (W.ARRAY, []))], [("t", W.T_F32, [1], bytes(4))]),
    }
    for what, (meta, tensors) in cases.items():
        b = W.gguf_bytes(meta, tensors)
        with pytest.raises(AfError):
            GgufInspector().inspect(write(tmp_path, "c.gguf", b))
        assert what  # (the case name documents the rejection)
    # an unknown tensor type id
    b = bytearray(W.gguf_bytes([], [("t", W.T_F32, [1], bytes(4))]))
    b[b.index(b"t") + 1 + 4 + 8] = 7
    with pytest.raises(AfError):
        GgufInspector().inspect(write(tmp_path, "u.gguf", bytes(b)))


def test_metadata_kinds_and_summarised_arrays(tmp_path):
    meta = [("u8", W.U8, 200), ("i8", W.I8, -5), ("u16", W.U16, 60000), ("i16", W.I16, -30000),
            ("u32", W.U32, 4000000000), ("i32", W.I32, -7), ("f32", W.F32, 0.5), ("bool", W.BOOL, True),
            ("text", W.STRING, "Gemma é"), ("u64", W.U64, 1 << 40), ("i64", W.I64, -(1 << 40)),
            ("f64", W.F64, 1e-300), ("small", W.ARRAY, (W.I32, [1, -2, 3])),
            ("big", W.ARRAY, (W.U8, list(range(256)) * 20))]
    p = write(tmp_path, "meta.gguf", W.gguf_bytes(meta, [("t", W.T_F32, [2], np.float32([1, 2]).tobytes())]))
    m = GgufInspector().inspect(p)
    want = {"u8": 200, "i8": -5, "u16": 60000, "i16": -30000, "u32": 4000000000, "i32": -7, "f32": 0.5,
            "bool": True, "text": "Gemma é", "u64": 1 << 40, "i64": -(1 << 40), "f64": 1e-300,
            "small": [1, -2, 3]}
    for k, v in want.items():
        assert m.metadata[k] == v, k
    assert m.metadata["big"] == ArraySummary(W.U8, 5120)
    assert np.array_equal(GgufInspector().read_f32_vector(p, "t"), np.float32([1, 2]))
    # invalid UTF-8 in a key is rejected
    b = W.gguf_bytes([("ok", W.U8, 1)], [("t", W.T_F32, [1], bytes(4))]).replace(b"ok", b"o\xff")
    with pytest.raises(AfError):
        GgufInspector().inspect(write(tmp_path, "utf.gguf", b))


@pytest.fixture(scope="module")
def gemma4_file(tmp_path_factory):
    model = synth.gemma4_model(name="gemma4-gguf", layers=6, hidden=512, intermediate=1024, local_q=(4, 2, 256),
                               global_q=(4, 1, 512), vocabulary=1024, window=8)
    path = str(tmp_path_factory.mktemp("gguf") / "gemma4.gguf")
    with open(path, "wb") as f:
        f.write(W.gemma4_gguf(model))
    return model, path


def test_synthetic_gemma4_file_round_trips_every_tensor(gemma4_file):
    model, path = gemma4_file
    ins = GgufInspector()
    info = ins.inspect(path)
    assert info.metadata["general.architecture"] == "gemma4" and info.metadata["gemma4.block_count"] == 6
    assert info.metadata["gemma4.attention.sliding_window_pattern"] == [True] * 5 + [False]
    assert info.data_offset % 32 == 0 and all(t.file_offset % 32 == 0 for t in info.tensors)
    names = {t.name for t in info.tensors}
    assert "blk.5.attn_v.weight" not in names and "blk.4.attn_v.weight" in names  # K reused as V on the global layer
    L5 = model.layers[5]
    q = ins.read_q4_matrix(path, "blk.5.attn_q.weight")
    assert (q.columns, q.rows) == (512, 4 * 512) and np.array_equal(q.data, L5.q)
    t = ins.read_q6_matrix(path, "token_embd.weight")
    assert (t.columns, t.rows) == (512, 1024) and np.array_equal(t.data, model.table)
    n = ins.read_rms_norm(path, "blk.5.attn_q_norm.weight")
    assert np.array_equal(n.weights, L5.q_norm) and n.epsilon == np.float32(1e-6)
    assert np.array_equal(ins.read_f32_vector(path, "rope_freqs.weight"), L5.rope_factors)
    width, vocab, ids, rows = ins.read_embeddings(path, [3, 1000])
    assert (width, vocab, ids) == (512, 1024, [3, 1000])
    row = 2 * 210
    assert np.array_equal(rows, np.concatenate([model.table[3 * row:4 * row], model.table[1000 * row:1001 * row]]))
    with pytest.raises(AfError):
        ins.read_embeddings(path, [1024])
    with pytest.raises(AfError):
        ins.read_q4_matrix(path, "token_embd.weight")  # wrong type
    with GgufFile(path) as g:
        with pytest.raises(AfError):
            g.read("blk.0.attn_norm.weight", 0, 512 * 4 + 1)  # past the tensor


def test_truncated_gemma4_file_is_rejected(gemma4_file, tmp_path):
    _, path = gemma4_file
    data = open(path, "rb").read()
    with pytest.raises(AfError):
        GgufInspector().inspect(write(tmp_path, "cut.gguf", data[:-1]))
    assert os.path.getsize(path) == len(data)
