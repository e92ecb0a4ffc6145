"""Python mirror of TVdxGGUFReader (src/VindexLLM.GGUFReader.pas:107-186)
over the library's GGUF reader (include/vdx_sampler.h, vdx_gguf_*).

The reader exists here for the lm_head's inputs: ``token_embd.weight`` (the
tied output projection, Model.Gemma3.pas:180-198), ``output_norm.weight``
(Model.Gemma3.pas:174) and the model dimensions in the metadata.  Parsing is
native (memory-mapped, bounds-checked); the methods keep the reference's
names, arguments and return conventions:

* ``Open`` returns False on a malformed or missing file, with a fatal entry
  in ``GetErrors()`` carrying the reference's code (GG02 bad magic, GG03
  version, GG01 parse, VF02 missing file; GGUFReader.pas:24-30, 376-430).
  Missing metadata and tensors are silent (False / default / None), as in
  the reference; ``GetTensorDataPtr`` on a missing tensor logs GG05.
* ``GetMetadataUInt64/UInt32/Float32/String`` return the default when the key
  is absent; a key of another type reads as the reference's zero-initialised
  field (0, 0.0 or '': ReadMetaValue fills only the field of its own type,
  GGUFReader.pas:542-600).
* ``GetTensorDataPtr`` returns the host address inside the mapping (None when
  the tensor is absent or its bytes run past the end of the file).

``tensor_bytes`` and ``tensor_to_device`` go beyond the reference: a read-only
numpy view of a tensor's bytes (it keeps the mapping alive) and a copy of them
into device memory in the GGUF layout that ``lmhead`` consumes.
``lm_head_from_gguf`` gathers what ``lmhead`` / ``TVdxSampler.lmhead_device``
need from a model file.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

from .sampler import (VDX_E_INVALID_ARG, VDX_E_UNSUPPORTED, VDX_OK, VDX_TENSOR_F16,
                      VDX_TENSOR_Q4_0, VDX_TENSOR_Q8_0, _GGUFInfo, _GGUFTensor, load_library)

# TVdxGGUFMetaType (GGUFReader.pas:71-85)
GMT_UINT8, GMT_INT8, GMT_UINT16, GMT_INT16, GMT_UINT32, GMT_INT32 = 0, 1, 2, 3, 4, 5
GMT_FLOAT32, GMT_BOOL, GMT_STRING, GMT_ARRAY = 6, 7, 8, 9
GMT_UINT64, GMT_INT64, GMT_FLOAT64 = 10, 11, 12

_UNSIGNED = (GMT_UINT8, GMT_UINT16, GMT_UINT32, GMT_UINT64)
_SIGNED = (GMT_INT8, GMT_INT16, GMT_INT32, GMT_INT64)
_FLOATS = (GMT_FLOAT32, GMT_FLOAT64)

# TVdxGGMLType names for the ids the reader sizes (GGUFReader.pas:34-67)
GGML_TYPE_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0",
                   9: "Q8_1", 10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K",
                   15: "Q8_K", 24: "I8", 25: "I16", 26: "I32", 27: "I64", 28: "F64", 30: "BF16"}

# the lm_head formats of the library (the reference's unembedding matvec
# handles these three, Attention.pas:1049-1066)
LMHEAD_TYPES = (VDX_TENSOR_F16, VDX_TENSOR_Q4_0, VDX_TENSOR_Q8_0)


@dataclass
class TVdxGGUFTensorInfo:
    """TVdxGGUFTensorInfo (GGUFReader.pas:98-104) plus the byte size
    (VdxGGMLTensorBytes, :264-318; 0 for types it does not size) and the
    absolute file offset."""
    TensorName: str
    NumDimensions: int
    Dimensions: list = field(default_factory=list)
    TensorType: int = 0
    DataOffset: int = 0      # relative to the data section, as in the file
    NBytes: int = 0
    FileOffset: int = 0


@dataclass
class TVdxGGUFMetaValue:
    """TVdxGGUFMetaValue (GGUFReader.pas:87-96); array items are not kept,
    only their type and count."""
    ValueType: int
    AsUInt64: int = 0
    AsInt64: int = 0
    AsFloat64: float = 0.0
    AsBool: bool = False
    AsString: str = ""
    ArrayType: int = 0
    ArrayLength: int = 0


@dataclass
class TVdxError:
    """One entry of the reader's error list (TVdxError, Utils.pas): severity
    'fatal' or 'error', the reference's code (GG01..GG06, VF02..VF06) and the
    message."""
    Severity: str
    Code: str
    Message: str


class TVdxErrors(list):
    def HasFatal(self) -> bool:
        return any(e.Severity == "fatal" for e in self)

    def HasErrors(self) -> bool:
        return len(self) > 0

    def GetItems(self):
        return list(self)


def _entry(severity: str, msg: bytes) -> TVdxError:
    text = msg.decode("utf-8", "replace") if msg else "gguf: error"
    code = text[:4] if len(text) > 5 and text[4] == ":" else ""
    return TVdxError(severity, code, text[6:] if code else text)


class _Mapping:
    """Owns one vdx_gguf handle; closed when the last user (the reader or a
    view from ``tensor_bytes``) lets go of it."""

    def __init__(self, h):
        self.h = h

    def close(self):
        if self.h:
            load_library().vdx_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _enc(s: str) -> bytes:
    # names and keys round-trip byte for byte, valid UTF-8 or not
    return s.encode("utf-8", "surrogateescape")


def _cstr(fn, *args) -> str:
    cap = 256
    while True:
        buf = C.create_string_buffer(cap)
        n = fn(*args, buf, cap)
        if n < 0:
            return None
        if n < cap:
            return buf.value.decode("utf-8", "surrogateescape")
        cap = n + 1


class TVdxGGUFReader:
    """TVdxGGUFReader (GGUFReader.pas:107-186) over the native reader."""

    def __init__(self):
        load_library()
        self._m = None
        self._errors = TVdxErrors()
        self._info = None

    # -- lifetime ---------------------------------------------------------
    def Open(self, path: str) -> bool:
        self.Close()
        L = load_library()
        h = C.c_void_p()
        rc = L.vdx_gguf_open(C.byref(h), str(path).encode())
        if rc != VDX_OK:
            self._errors.append(_entry("fatal", L.vdx_gguf_last_error(None)))
            return False
        self._m = _Mapping(h)
        info = _GGUFInfo()
        L.vdx_gguf_get_info(h, C.byref(info))
        self._info = info
        return True

    def Close(self):
        """Drops this reader's hold on the mapping; views from
        ``tensor_bytes`` keep it alive until they are released."""
        if self._m is not None:
            self._m = None
        self._info = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.Close()

    def IsOpen(self) -> bool:
        return self._m is not None

    def GetErrors(self) -> TVdxErrors:
        return self._errors

    def _h(self):
        if self._m is None:
            raise RuntimeError("gguf: reader is not open")
        return self._m.h

    def _fail(self):
        self._errors.append(_entry("error", load_library().vdx_gguf_last_error(self._h())))

    # -- header -----------------------------------------------------------
    def GetVersion(self) -> int:
        return int(self._info.version) if self._info else 0

    def GetTensorCount(self) -> int:
        return int(self._info.tensor_count) if self._info else 0

    def GetMetadataCount(self) -> int:
        return int(self._info.metadata_count) if self._info else 0

    def GetAlignment(self) -> int:
        return int(self._info.alignment) if self._info else 0

    def GetFileSize(self) -> int:
        return int(self._info.file_size) if self._info else 0

    def GetDataOffset(self) -> int:
        return int(self._info.data_offset) if self._info else 0

    # -- metadata ---------------------------------------------------------
    def _type(self, key: str) -> int:
        if self._m is None:
            return VDX_E_INVALID_ARG
        return load_library().vdx_gguf_meta_type(self._h(), _enc(key))

    def HasMetadata(self, key: str) -> bool:
        return self._type(key) >= 0

    def GetMetadata(self, key: str):
        """(found, TVdxGGUFMetaValue) like GetMetadata's Boolean + out value."""
        t = self._type(key)
        if t < 0:
            return False, TVdxGGUFMetaValue(ValueType=0)
        L, h, k = load_library(), self._h(), _enc(key)
        v = TVdxGGUFMetaValue(ValueType=t)
        if t in _UNSIGNED or t in _SIGNED or t == GMT_BOOL:
            x = C.c_int64()
            L.vdx_gguf_meta_int(h, k, C.byref(x))
            if t in _UNSIGNED:
                v.AsUInt64 = x.value & 0xFFFFFFFFFFFFFFFF
            elif t in _SIGNED:
                v.AsInt64 = x.value
            else:
                v.AsBool = bool(x.value)
        elif t in _FLOATS:
            x = C.c_double()
            L.vdx_gguf_meta_float(h, k, C.byref(x))
            v.AsFloat64 = x.value
        elif t == GMT_STRING:
            v.AsString = _cstr(L.vdx_gguf_meta_string, h, k)
        elif t == GMT_ARRAY:
            et, n = C.c_int32(), C.c_int64()
            L.vdx_gguf_meta_array(h, k, C.byref(et), C.byref(n))
            v.ArrayType, v.ArrayLength = et.value, n.value
        return True, v

    def GetMetadataString(self, key: str, default: str = "") -> str:
        ok, v = self.GetMetadata(key)
        return v.AsString if ok else default

    def GetMetadataUInt64(self, key: str, default: int = 0) -> int:
        ok, v = self.GetMetadata(key)
        return v.AsUInt64 if ok else default

    def GetMetadataUInt32(self, key: str, default: int = 0) -> int:
        ok, v = self.GetMetadata(key)
        return (v.AsUInt64 & 0xFFFFFFFF) if ok else default

    def GetMetadataFloat32(self, key: str, default: float = 0.0) -> float:
        import numpy as np
        ok, v = self.GetMetadata(key)
        return float(np.float32(v.AsFloat64)) if ok else default

    def GetMetadataKeys(self):
        if self._m is None:
            return []
        L, h = load_library(), self._h()
        out, i = [], 0
        while True:
            k = _cstr(L.vdx_gguf_meta_key, h, i)
            if k is None:
                return out
            out.append(k)
            i += 1

    def GetArrayLength(self, key: str) -> int:
        """Element count of an array value (0 when absent or not an array);
        tokenizer.ggml.tokens gives the vocabulary size (Tokenizer.pas:124)."""
        ok, v = self.GetMetadata(key)
        return v.ArrayLength if ok and v.ValueType == GMT_ARRAY else 0

    # -- tensors ----------------------------------------------------------
    def _find(self, name: str):
        t = _GGUFTensor()
        if self._m is None:
            return VDX_E_INVALID_ARG, t
        rc = load_library().vdx_gguf_find_tensor(self._h(), _enc(name), C.byref(t))
        return rc, t

    def HasTensor(self, name: str) -> bool:
        return self._find(name)[0] != VDX_E_INVALID_ARG

    def GetTensorInfo(self, name: str):
        """TVdxGGUFTensorInfo, or None when the file holds no such tensor."""
        rc, t = self._find(name)
        if rc == VDX_E_INVALID_ARG:
            return None
        return TVdxGGUFTensorInfo(
            TensorName=name, NumDimensions=t.n_dims, Dimensions=[int(t.dims[d]) for d in range(t.n_dims)],
            TensorType=t.type, DataOffset=int(t.file_offset) - self.GetDataOffset(),
            NBytes=int(t.nbytes), FileOffset=int(t.file_offset))

    def GetTensorDataPtr(self, name: str):
        if self._m is None:
            self._errors.append(TVdxError("error", "GG06", "GGUF file not open"))
            return None
        rc, t = self._find(name)
        if rc != VDX_OK:
            self._fail()
            return None
        return t.data

    def GetTensorList(self):
        if self._m is None:
            return []
        L, h = load_library(), self._h()
        names = [_cstr(L.vdx_gguf_tensor_name, h, i) for i in range(self.GetTensorCount())]
        return [self.GetTensorInfo(n) for n in names]

    def tensor_bytes(self, name: str):
        """Read-only numpy uint8 view of the tensor's bytes in the mapping."""
        import numpy as np
        rc, t = self._find(name)
        if rc != VDX_OK:
            self._fail()
            raise KeyError(self._errors[-1].Message)
        if t.nbytes == 0:
            raise ValueError(f"gguf: tensor '{name}' has type {GGML_TYPE_NAMES.get(t.type, t.type)}, "
                             "which the reader does not size")
        buf = (C.c_uint8 * int(t.nbytes)).from_address(t.data)
        buf._mapping = self._m
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a

    def tensor_to_device(self, name: str, device):
        """The tensor's bytes, unchanged, in a uint8 torch tensor on `device`."""
        import torch
        src = torch.from_numpy(self.tensor_bytes(name).copy())
        return src.to(device)


def lm_head_from_gguf(reader: TVdxGGUFReader, device, norm: bool = True, pack: bool = False):
    """What the lm_head needs from a model file, on `device`:

    weights    token_embd.weight in its GGUF layout (uint8), the tied output
               projection (Model.Gemma3.pas:180-198)
    wtype      its GGML type (F16, Q4_0 or Q8_0)
    in_dim     the hidden size (the row length, Dimensions[0])
    vocab      the number of rows (Dimensions[1])
    norm_weight output_norm.weight as float32 (Model.Gemma3.pas:174, read as
               in_dim singles like UploadNormWeight, Model.pas:514-540), or
               None when `norm` is False
    norm_eps   1e-6, the reference's RMSNorm epsilon (LayerNorm.pas:186)

    With ``pack`` the weights are repacked on the device (``lmhead_pack``)
    and ``wtype`` carries VDX_LMHEAD_PACKED.
    """
    import numpy as np
    import torch
    info = reader.GetTensorInfo("token_embd.weight")
    if info is None:
        raise KeyError("gguf: token_embd.weight not found")
    if info.TensorType not in LMHEAD_TYPES:
        raise ValueError("gguf: token_embd.weight has type %s; the lm_head takes F16, Q4_0 or Q8_0"
                         % GGML_TYPE_NAMES.get(info.TensorType, info.TensorType))
    if info.NumDimensions != 2:
        raise ValueError(f"gguf: token_embd.weight has {info.NumDimensions} dimensions")
    in_dim, vocab = info.Dimensions
    out = dict(weights=reader.tensor_to_device("token_embd.weight", device), wtype=info.TensorType,
               in_dim=int(in_dim), vocab=int(vocab), norm_weight=None, norm_eps=1e-6)
    if pack:
        from .sampler import VDX_LMHEAD_PACKED, lmhead_pack
        out["weights"] = lmhead_pack(out["weights"], info.TensorType, int(in_dim), int(vocab))
        out["wtype"] = info.TensorType | VDX_LMHEAD_PACKED
    if norm:
        ninfo = reader.GetTensorInfo("output_norm.weight")
        if ninfo is None:
            raise KeyError("gguf: output_norm.weight not found")
        raw = reader.tensor_bytes("output_norm.weight")
        if raw.size < 4 * in_dim:
            raise ValueError("gguf: output_norm.weight holds fewer than in_dim singles")
        w = np.frombuffer(raw[:4 * in_dim].tobytes(), dtype=np.float32)
        out["norm_weight"] = torch.from_numpy(w.copy()).to(device)
    return out


__all__ = ["TVdxGGUFReader", "TVdxGGUFTensorInfo", "TVdxGGUFMetaValue", "TVdxError", "lm_head_from_gguf",
           "GGML_TYPE_NAMES", "LMHEAD_TYPES", "VDX_E_UNSUPPORTED"]
