"""The whole-model upload's host side, CPU only: the GGUF container reader/writer of the harness
against the reference's own MappedGgufModel (compiled from its sources, where oracle/_ref is
built), and oq_model_validate's checks -- the reference's, in its order
(src/model/mapped_gguf.cpp:124-203, src/model/ggml_type.cpp:96-118) -- with the same error kinds."""
import numpy as np
import pytest

import oracle
import oracle_amd
from oracle_amd import gguf, synth


def model_tensors(rng):
    """A mixed table: matrices of every multiplied type, vectors, a registered type without a
    device decoder (q4_0), a rank-3 tensor."""
    out = []
    for name, t, rows, cols in (("blk.0.ffn_gate.weight", 12, 40, 512), ("blk.0.ffn_up.weight", 13, 33, 768),
                                ("blk.0.attn_output.weight", 14, 17, 256), ("token_embd.weight", 8, 9, 96),
                                ("blk.0.ssm_out.weight", 0, 5, 33), ("blk.0.attn_q.weight", 1, 7, 130),
                                ("output.weight", 30, 6, 64)):
        if t in (12, 13, 14, 8):
            data = synth.weights(t, rng, rows, cols)
        elif t == 0:
            data = rng.standard_normal(rows * cols).astype(np.float32).view(np.uint8)
        elif t == 1:
            data = rng.standard_normal(rows * cols).astype(np.float16).view(np.uint8)
        else:
            data = (rng.standard_normal(rows * cols).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
        out.append((name, [cols, rows], t, data))
    out.append(("blk.0.attn_norm.weight", [512], 0, rng.standard_normal(512).astype(np.float32).view(np.uint8)))
    out.append(("blk.0.ssm_conv1d.weight", [4, 24], 0, rng.standard_normal(96).astype(np.float32).view(np.uint8)))
    out.append(("blk.0.q4_0.weight", [64, 3], 2, np.frombuffer(rng.bytes(3 * 2 * 18), np.uint8).copy()))
    out.append(("blk.0.experts.weight", [8, 4, 2], 0, rng.standard_normal(64).astype(np.float32).view(np.uint8)))
    return out


def test_reader_matches_writer(tmp_path):
    rng = np.random.default_rng(1)
    tensors = model_tensors(rng)
    path = tmp_path / "m.gguf"
    gguf.write(path, tensors, {"general.name": "fixture"})
    f = gguf.read(path)
    assert f.version == 3 and f.metadata["general.name"] == "fixture" and f.data_offset % 32 == 0
    payload = f.payload()
    for (name, dims, t, data), info in zip(tensors, f.tensors):
        assert (info.name, info.dims, info.type) == (name, dims, t)
        assert info.absolute_offset % 32 == 0
        assert np.array_equal(payload[info.absolute_offset:info.absolute_offset + data.nbytes], data)
    oracle_amd.model_validate(f.file_size, [(t.name, t.dims, t.type, t.absolute_offset) for t in f.tensors])


@pytest.mark.skipif(not oracle.ref_available(), reason="compiled reference (oracle/_ref) not built here")
def test_reader_matches_reference_mapping(tmp_path):
    rng = np.random.default_rng(2)
    tensors = model_tensors(rng)
    path = tmp_path / "m.gguf"
    gguf.write(path, tensors, {"general.name": "fixture"}, alignment=64)
    f = gguf.read(path)
    ref = oracle.ref_gguf_tensors(path)
    assert [(r["name"], r["type"], r["dims"], r["absolute_offset"]) for r in ref] == \
        [(t.name, t.type, t.dims, t.absolute_offset) for t in f.tensors]
    for r, (_, _, _, data) in zip(ref, tensors):
        assert r["nbytes"] == data.nbytes


def test_validate_rejects_like_the_reference():
    ok = [("a", [256, 2], 12, 0), ("b", [32], 0, 288)]
    oracle_amd.model_validate(416, ok)
    cases = [
        ([("a", [256, 2], 4, 0)], oracle_amd.UnsupportedType, "unsupported GGML tensor type 4 for tensor a"),
        ([("a", [256, 0], 12, 0)], oracle_amd.OqError, "GGUF tensor dimensions must be non-zero"),
        ([("a", [256, 2], 12, 500)], oracle_amd.OqError, "GGUF tensor offset exceeds file size: a"),
        ([("a", [100, 2], 12, 0)], oracle_amd.UnsupportedType, "not divisible by block size"),
        ([("a", [1 << 40, 1 << 40], 0, 0)], oracle_amd.Overflow, "overflow"),
        ([("a", [256, 2], 12, 200)], oracle_amd.OqError, "payload exceeds file size: a"),
        ([("a", [256, 2], 12, 0), ("a", [32], 0, 288)], oracle_amd.OqError, "duplicate GGUF tensor name: a"),
        ([("a", [256, 2], 12, 0), ("b", [32], 0, 128)], oracle_amd.OqError, "payloads overlap: a and b"),
    ]
    for table, kind, text in cases:
        with pytest.raises(kind) as e:
            oracle_amd.model_validate(416, table)
        assert text in str(e.value), (text, str(e.value))


@pytest.mark.skipif(not oracle.ref_available(), reason="compiled reference (oracle/_ref) not built here")
def test_reference_rejects_the_same_files(tmp_path):
    """Malformed files: the reference's MappedGgufModel and oq_model_validate reject them with
    the same message."""
    rng = np.random.default_rng(3)
    a = ("a", [256, 2], 12, synth.q4_k(rng, 2, 256))
    b = ("b", [32], 0, rng.standard_normal(32).astype(np.float32).view(np.uint8))
    for label, tensors, offsets, text in (
            ("overlap", [a, b], [0, 128], "overlap"),
            ("duplicate", [a, ("a", [32], 0, b[3])], None, "duplicate GGUF tensor name: a"),
            ("beyond", [a, b], [0, 1 << 20], "offset exceeds file size: b"),
            ("end_beyond", [a, ("b", [4096], 0, b[3])], None, "payload exceeds file size: b")):
        path = tmp_path / f"{label}.gguf"
        gguf.write(path, tensors, offsets=offsets)
        with pytest.raises(oracle.OracleError) as e:
            oracle.ref_gguf_tensors(path)
        assert text in str(e.value), str(e.value)
        f = gguf.read(path)
        with pytest.raises(oracle_amd.OqError) as e2:
            oracle_amd.model_validate(f.file_size, [(t.name, t.dims, t.type, t.absolute_offset) for t in f.tensors])
        assert text in str(e2.value)
