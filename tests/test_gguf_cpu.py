"""GGUF reader (vdx_gguf_* in libvdxsampler.so, vindexllm_amd.gguf) on
synthetic model files written by tests/ggufw.py.

The reference's own reader tests (testbed/UTest.GGUFReader.pas) open a Gemma
3 model at a fixed Windows path, which is not here; their sections are ported
onto synthetic files: initial state, missing file (VF02), bad magic (GG02),
header fields, metadata and tensor lookups, silent misses, Close and reopen.
Beyond them: every metadata value type, nested arrays, the alignment rule,
tensor byte sizes (VdxGGMLTensorBytes, GGUFReader.pas:264-318), and every
truncation and a byte-flip sweep of a small file, which must end in an error
and never a fault.  Parsing only; no GPU.
"""
import os
import struct

import numpy as np
import pytest

import ggufw as W
from vindexllm_amd import gguf as G
from vindexllm_amd.gguf import TVdxGGUFReader, lm_head_from_gguf


def _q4_0(rng, rows, in_dim):
    nb = in_dim // 32
    blk = np.zeros((rows, nb, 18), dtype=np.uint8)
    d = np.abs(rng.standard_normal((rows, nb)) * 0.02).astype(np.float16)
    blk[:, :, 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:] = rng.integers(0, 256, (rows, nb, 16), dtype=np.uint8)
    return blk.reshape(-1).tobytes()


IN_DIM, VOCAB = 128, 96


def _model(rng, embd_type=2, alignment=None, extra_meta=(), version=3):
    if embd_type == 2:
        embd = _q4_0(rng, VOCAB, IN_DIM)
    elif embd_type == 8:
        embd = rng.integers(0, 256, VOCAB * IN_DIM // 32 * 34, dtype=np.uint8).tobytes()
    else:
        embd = (rng.standard_normal(VOCAB * IN_DIM) * 0.1).astype(np.float16).tobytes()
    norm = (1.0 + rng.standard_normal(IN_DIM) * 0.1).astype(np.float32).tobytes()
    meta = [("general.architecture", W.STR, "gemma3"),
            ("general.name", W.STR, "synthetic"),
            ("gemma3.embedding_length", W.U32, IN_DIM),
            ("gemma3.block_count", W.U32, 2),
            ("gemma3.attention.layer_norm_rms_epsilon", W.F32, 1e-6),
            ("tokenizer.ggml.tokens", W.ARR, (W.STR, ["t%d" % i for i in range(VOCAB)])),
            ("tokenizer.ggml.scores", W.ARR, (W.F32, [0.5] * VOCAB))]
    if alignment is not None:
        meta.append(("general.alignment", W.U32, alignment))
    meta += list(extra_meta)
    tensors = [("output_norm.weight", [IN_DIM], 0, norm),
               ("token_embd.weight", [IN_DIM, VOCAB], embd_type, embd),
               ("blk.0.attn_q.weight", [IN_DIM, 64], 1,
                rng.standard_normal(IN_DIM * 64).astype(np.float16).tobytes())]
    blob, offs = W.build(meta, tensors, version=version, alignment=alignment)
    return blob, offs, dict(embd=embd, norm=norm)


def _write(tmp_path, blob, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(blob)
    return str(p)


def test_initial_state_and_missing_file(tmp_path):
    # UTest.GGUFReader.pas: SecInitialState, SecOpenMissingFile
    r = TVdxGGUFReader()
    assert not r.GetErrors().HasFatal()
    assert (r.GetVersion(), r.GetTensorCount(), r.GetMetadataCount(), r.GetFileSize()) == (0, 0, 0, 0)
    assert not r.Open(str(tmp_path / "does_not_exist.gguf"))
    assert r.GetErrors().HasFatal()
    assert r.GetErrors().GetItems()[0].Code == "VF02"
    empty = _write(tmp_path, b"", "empty.gguf")
    r2 = TVdxGGUFReader()
    assert not r2.Open(empty) and r2.GetErrors()[0].Code == "VF06"


def test_bad_magic_and_version(tmp_path):
    # SecOpenBadMagic: 'JUNK' then zeros, 32 bytes
    p = _write(tmp_path, b"JUNK" + b"\0" * 28, "bad_magic.gguf")
    r = TVdxGGUFReader()
    assert not r.Open(p)
    assert r.GetErrors().HasFatal() and any(e.Code == "GG02" for e in r.GetErrors())
    blob, _ = W.build([], [], version=1)
    r = TVdxGGUFReader()
    assert not r.Open(_write(tmp_path, blob, "v1.gguf"))
    assert r.GetErrors()[0].Code == "GG03"
    for v in (2, 3):
        blob, _ = W.build([("a", W.U8, 1)], [], version=v)
        r = TVdxGGUFReader()
        assert r.Open(_write(tmp_path, blob, "v%d.gguf" % v)) and r.GetVersion() == v


def test_header_metadata_tensors_close_reopen(tmp_path):
    rng = np.random.default_rng(1)
    blob, offs, data = _model(rng)
    p = _write(tmp_path, blob)
    r = TVdxGGUFReader()
    assert r.Open(p), r.GetErrors()
    # SecHeaderFields
    assert r.GetVersion() == 3 and r.GetTensorCount() == 3 and r.GetMetadataCount() == 7
    assert r.GetFileSize() == len(blob) and r.GetAlignment() == 32
    # SecMetadataLookup
    assert r.HasMetadata("general.architecture")
    ok, v = r.GetMetadata("general.architecture")
    assert ok and v.ValueType == G.GMT_STRING and v.AsString == "gemma3"
    assert r.GetMetadataString("general.architecture") == "gemma3"
    assert r.GetMetadataUInt32("gemma3.embedding_length") == IN_DIM
    assert r.GetMetadataFloat32("gemma3.attention.layer_norm_rms_epsilon") == float(np.float32(1e-6))
    assert r.GetArrayLength("tokenizer.ggml.tokens") == VOCAB
    ok, v = r.GetMetadata("tokenizer.ggml.scores")
    assert ok and v.ValueType == G.GMT_ARRAY and v.ArrayType == G.GMT_FLOAT32 and v.ArrayLength == VOCAB
    assert sorted(r.GetMetadataKeys()) == sorted(
        ["general.architecture", "general.name", "gemma3.embedding_length", "gemma3.block_count",
         "gemma3.attention.layer_norm_rms_epsilon", "tokenizer.ggml.tokens", "tokenizer.ggml.scores"])
    # SecTensorLookup
    assert r.HasTensor("token_embd.weight")
    info = r.GetTensorInfo("token_embd.weight")
    assert info.NumDimensions == 2 and info.Dimensions == [IN_DIM, VOCAB] and info.TensorType == 2
    assert info.NBytes == VOCAB * IN_DIM // 32 * 18 == len(data["embd"])
    assert info.FileOffset == offs["token_embd.weight"] and info.FileOffset % 32 == 0
    assert info.DataOffset == info.FileOffset - r.GetDataOffset()
    assert r.GetTensorDataPtr("token_embd.weight")
    assert r.tensor_bytes("token_embd.weight").tobytes() == data["embd"]
    assert r.tensor_bytes("output_norm.weight").tobytes() == data["norm"]
    lst = r.GetTensorList()
    assert [t.TensorName for t in lst] == ["output_norm.weight", "token_embd.weight", "blk.0.attn_q.weight"]
    assert lst[2].NBytes == IN_DIM * 64 * 2
    # SecMissingMetadata / SecMissingTensor: silent
    assert not r.HasMetadata("this.key.does.not.exist")
    assert r.GetMetadata("this.key.does.not.exist")[0] is False
    assert r.GetMetadataString("this.key.does.not.exist", "fallback-value") == "fallback-value"
    assert r.GetMetadataUInt32("this.key.does.not.exist", 7) == 7
    assert not r.HasTensor("this.tensor.does.not.exist")
    assert r.GetTensorInfo("this.tensor.does.not.exist") is None
    assert not r.GetErrors().HasFatal() and not r.GetErrors().HasErrors()
    assert r.GetTensorDataPtr("this.tensor.does.not.exist") is None
    assert r.GetErrors()[-1].Code == "GG05" and not r.GetErrors().HasFatal()
    # SecClose: reset, idempotent, reopen
    view = r.tensor_bytes("token_embd.weight")
    r.Close()
    assert (r.GetTensorCount(), r.GetMetadataCount(), r.GetFileSize()) == (0, 0, 0)
    r.Close()
    assert not r.GetErrors().HasFatal()
    assert view.tobytes() == data["embd"]  # a view keeps the mapping alive
    del view
    assert r.Open(p) and r.GetTensorCount() == 3


def test_every_metadata_type_and_the_reference_field_rule(tmp_path):
    meta = [("u8", W.U8, 250), ("i8", W.I8, -5), ("u16", W.U16, 65000), ("i16", W.I16, -30000),
            ("u32", W.U32, 4_000_000_000), ("i32", W.I32, -2_000_000_000), ("f32", W.F32, 1.5),
            ("b", W.BOOL, 1), ("s", W.STR, "héllo"), ("u64", W.U64, 2**64 - 3),
            ("i64", W.I64, -2**62), ("f64", W.F64, 0.1),
            ("nested", W.ARR, (W.ARR, [(W.U8, [1, 2, 3]), (W.STR, ["a", "bc"])])),
            ("strs", W.ARR, (W.STR, ["x", "", "yz"])), ("empty", W.ARR, (W.I32, []))]
    blob, _ = W.build(meta, [])
    r = TVdxGGUFReader()
    assert r.Open(_write(tmp_path, blob)), r.GetErrors()
    assert r.GetMetadataCount() == len(meta)
    assert r.GetMetadataUInt64("u8") == 250 and r.GetMetadataUInt64("u16") == 65000
    assert r.GetMetadataUInt64("u32") == 4_000_000_000 and r.GetMetadataUInt64("u64") == 2**64 - 3
    assert r.GetMetadataUInt32("u64") == (2**64 - 3) & 0xFFFFFFFF
    assert r.GetMetadata("i8")[1].AsInt64 == -5 and r.GetMetadata("i16")[1].AsInt64 == -30000
    assert r.GetMetadata("i32")[1].AsInt64 == -2_000_000_000 and r.GetMetadata("i64")[1].AsInt64 == -2**62
    assert r.GetMetadata("b")[1].AsBool is True
    assert r.GetMetadataFloat32("f32") == 1.5 and r.GetMetadata("f64")[1].AsFloat64 == 0.1
    assert r.GetMetadataFloat32("f64") == float(np.float32(0.1))
    assert r.GetMetadataString("s") == "héllo"
    ok, v = r.GetMetadata("nested")
    assert ok and v.ArrayType == G.GMT_ARRAY and v.ArrayLength == 2
    assert r.GetArrayLength("strs") == 3 and r.GetArrayLength("empty") == 0
    # ReadMetaValue fills only its own type's field (GGUFReader.pas:542-600):
    # the typed getters read the zero of the others
    assert r.GetMetadataUInt64("i32") == 0 and r.GetMetadataUInt32("b") == 0
    assert r.GetMetadataFloat32("u32") == 0.0 and r.GetMetadataString("u8") == ""


def test_alignment_rule(tmp_path):
    rng = np.random.default_rng(2)
    for align in (64, 48, 1, 4096):
        blob, offs, data = _model(rng, alignment=align)
        r = TVdxGGUFReader()
        assert r.Open(_write(tmp_path, blob, "a%d.gguf" % align)), r.GetErrors()
        assert r.GetAlignment() == align and r.GetDataOffset() % align == 0
        for name, off in offs.items():
            assert r.GetTensorInfo(name).FileOffset == off and off % align == 0
        assert r.tensor_bytes("token_embd.weight").tobytes() == data["embd"]
    # zero, a signed type, and the key in another case (SameText)
    for meta, want in ((("general.alignment", W.U32, 0), 32), (("general.alignment", W.I32, 64), 32),
                       (("GENERAL.Alignment", W.U64, 128), 128)):
        blob, _ = W.build([meta], [("x", [32], 0, b"\1" * 128)], alignment=want)
        r = TVdxGGUFReader()
        assert r.Open(_write(tmp_path, blob, "z.gguf")) and r.GetAlignment() == want
        assert r.tensor_bytes("x").tobytes() == b"\1" * 128


def test_tensor_byte_sizes(tmp_path):
    # VdxGGMLTensorBytes (GGUFReader.pas:243-318) for each type it sizes;
    # 0 for the others (Q5_0 = 6 here)
    cases = {0: 4 * 256, 1: 2 * 256, 2: 256 // 32 * 18, 3: 256 // 32 * 20, 8: 256 // 32 * 34,
             12: 144, 13: 176, 14: 210, 24: 256, 25: 512, 26: 1024, 27: 2048, 28: 2048, 30: 512, 6: 0}
    tensors = [("t%d" % t, [128, 2], t, b"\0" * max(n, 1)) for t, n in cases.items()]
    blob, _ = W.build([], tensors)
    r = TVdxGGUFReader()
    assert r.Open(_write(tmp_path, blob)), r.GetErrors()
    for t, n in cases.items():
        assert r.GetTensorInfo("t%d" % t).NBytes == n, t
    with pytest.raises(ValueError):
        r.tensor_bytes("t6")


def test_tensor_past_end_and_wrapping_dims(tmp_path):
    rng = np.random.default_rng(3)
    blob, offs, _ = _model(rng)
    cut = offs["token_embd.weight"] + 100  # token_embd runs past the end
    r = TVdxGGUFReader()
    assert r.Open(_write(tmp_path, blob[:cut])), r.GetErrors()
    assert r.HasTensor("token_embd.weight")
    info = r.GetTensorInfo("token_embd.weight")
    assert info.Dimensions == [IN_DIM, VOCAB]
    assert r.GetTensorDataPtr("token_embd.weight") is None and r.GetErrors()[-1].Code == "GG05"
    with pytest.raises(KeyError):
        r.tensor_bytes("token_embd.weight")
    assert r.tensor_bytes("output_norm.weight").size == 4 * IN_DIM
    # dims whose product wraps 2^64 must not pass as a small tensor
    blob, _ = W.build([], [("w", [2**33, 2**31 + 1], 0, b"\0" * 64)])
    r = TVdxGGUFReader()
    assert r.Open(_write(tmp_path, blob, "w.gguf"))
    assert r.GetTensorDataPtr("w") is None


def _opens(path):
    r = TVdxGGUFReader()
    ok = r.Open(path)
    if not ok:
        assert r.GetErrors().HasFatal() and r.GetErrors()[0].Code in ("GG01", "GG02", "GG03", "VF06")
    return ok, r


def test_every_truncation_is_an_error_not_a_fault(tmp_path):
    rng = np.random.default_rng(4)
    blob, offs, _ = _model(rng)
    data_start = min(offs.values())
    p = str(tmp_path / "t.gguf")
    for n in range(0, data_start + 1):
        with open(p, "wb") as f:
            f.write(blob[:n])
        ok, r = _opens(p)
        # the directory ends before the padding to the data section; a file
        # cut inside the padding still parses (its data start is the aligned
        # offset, possibly past the end: then it is an error)
        if ok:
            assert n >= data_start - 31
            for name in offs:
                assert r.GetTensorDataPtr(name) is None


def test_corrupted_headers_are_errors(tmp_path):
    rng = np.random.default_rng(5)
    blob, offs, _ = _model(rng)
    p = str(tmp_path / "c.gguf")
    # implausible counts, a huge string length, 5 dims, unknown value types
    bad = [blob[:8] + struct.pack("<Q", 2**40) + blob[16:],
           blob[:16] + struct.pack("<Q", 2**40) + blob[24:]]
    key_len_at = 24
    bad.append(blob[:key_len_at] + struct.pack("<Q", 2**62) + blob[key_len_at + 8:])
    type_at = key_len_at + 8 + len("general.architecture")
    bad.append(blob[:type_at] + struct.pack("<I", 13) + blob[type_at + 4:])
    arr = W.build([("a", W.ARR, (W.U8, [1]))], [])[0]
    at = 24 + 8 + 1 + 4
    bad.append(arr[:at] + struct.pack("<I", 99) + arr[at + 4:])
    bad.append(W.build([], [("t", [1, 1, 1, 1, 1], 0, b"\0" * 4)])[0])
    bad.append(W.build([], [("t", [], 0, b"")])[0])
    for b in bad:
        with open(p, "wb") as f:
            f.write(b)
        ok, _ = _opens(p)
        assert not ok


def test_byte_flip_sweep_never_faults(tmp_path):
    # every byte of the header and directory replaced by 0xFF and by 0x7F in
    # turn: each file either parses or is refused, and a parsed one answers
    # every lookup without touching memory outside the mapping
    rng = np.random.default_rng(6)
    blob, offs, _ = _model(rng)
    data_start = min(offs.values())
    p = str(tmp_path / "f.gguf")
    parsed = 0
    for i in range(data_start):
        for x in (0xFF, 0x7F):
            b = bytearray(blob)
            b[i] = x
            with open(p, "wb") as f:
                f.write(b)
            ok, r = _opens(p)
            if ok:
                parsed += 1
                for t in r.GetTensorList():
                    ptr = r.GetTensorDataPtr(t.TensorName)
                    if ptr is not None and t.NBytes:
                        assert t.FileOffset + t.NBytes <= len(b)
                        r.tensor_bytes(t.TensorName).sum()
                r.GetMetadataKeys()
    assert parsed > 0


def test_duplicate_keys_keep_the_last_value(tmp_path):
    # AddOrSetValue (GGUFReader.pas:656): a repeated key keeps the last value
    blob, _ = W.build([("k", W.U32, 1), ("k", W.U32, 2)], [])
    r = TVdxGGUFReader()
    assert r.Open(_write(tmp_path, blob))
    assert r.GetMetadataCount() == 2 and r.GetMetadataKeys() == ["k"] and r.GetMetadataUInt32("k") == 2


@pytest.mark.parametrize("embd_type", [2, 8, 1])
def test_lm_head_inputs_from_gguf(tmp_path, embd_type):
    import torch
    rng = np.random.default_rng(7)
    blob, _, data = _model(rng, embd_type=embd_type, alignment=64)
    r = TVdxGGUFReader()
    assert r.Open(_write(tmp_path, blob))
    lm = lm_head_from_gguf(r, torch.device("cpu"))
    assert lm["wtype"] == embd_type and lm["in_dim"] == IN_DIM and lm["vocab"] == VOCAB
    assert lm["weights"].dtype == torch.uint8 and lm["weights"].numpy().tobytes() == data["embd"]
    assert lm["norm_weight"].dtype == torch.float32
    assert lm["norm_weight"].numpy().tobytes() == data["norm"] and lm["norm_eps"] == 1e-6


def test_lm_head_rejects_other_embedding_types(tmp_path):
    import torch
    blob, _ = W.build([], [("token_embd.weight", [64, 4], 0, b"\0" * 1024)])
    r = TVdxGGUFReader()
    assert r.Open(_write(tmp_path, blob))
    with pytest.raises(ValueError):
        lm_head_from_gguf(r, torch.device("cpu"))
    blob, _ = W.build([], [])
    r = TVdxGGUFReader()
    assert r.Open(_write(tmp_path, blob, "e.gguf"))
    with pytest.raises(KeyError):
        lm_head_from_gguf(r, torch.device("cpu"))

