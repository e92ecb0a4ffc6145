"""Python mirror of the reference sampler interface over libvdxsampler.so.

``TVdxSamplerConfig`` and ``TVdxSampler`` keep the names, argument meaning
and defaults of src/VindexLLM.Sampler.pas:26-91 (Create / SetConfig /
GetConfig / DefaultConfig / Process / AddToHistory / ResetHistory).  Every
call goes through the C ABI of include/vdx_sampler.h; sampling runs in the
library's HIP kernels on the GPU.  There is no CPU fallback: if the library
is not built, or no GPU is present, construction raises.

Beyond the reference (whose sampler holds one sequence), ``process_device``
samples a batch of device-resident rows (torch tensors on the GPU) without
moving logits to the host.
"""
from __future__ import annotations

import ctypes as C
import os

from . import build as _build

VDX_OK = 0
VDX_E_INVALID_ARG = -1
VDX_E_HIP = -2
VDX_E_UNSUPPORTED = -3
VDX_E_NO_MEMORY = -4

VDX_RNG_XOSHIRO = 0
VDX_RNG_PHILOX = 1

VDX_TENSOR_F16 = 1   # lm_head weight formats: GGML type ids (GGUFReader.pas:34-42)
VDX_TENSOR_Q4_0 = 2
VDX_TENSOR_Q8_0 = 8
VDX_LMHEAD_PACKED = 0x100  # OR-ed into wtype: weights in the layout of lmhead_pack

ROW_GREEDY = 0x1
ROW_TOPK_FAST = 0x2
ROW_TOPK_REPLAY = 0x4
ROW_FULL = 0x8
ROW_NAN = 0x10
ROW_FALLBACK = 0x20


class VdxSamplerError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"vdx_sampler error {code}: {msg}")
        self.code = code


class TVdxSamplerConfig(C.Structure):
    """TVdxSamplerConfig (Sampler.pas:26-34); 32 bytes like the {$A8} record."""

    _fields_ = [
        ("Temperature", C.c_float),
        ("TopK", C.c_int32),
        ("TopP", C.c_float),
        ("MinP", C.c_float),
        ("RepeatPenalty", C.c_float),
        ("RepeatWindow", C.c_int32),
        ("Seed", C.c_int64),
    ]

    def __repr__(self):
        return ("TVdxSamplerConfig(Temperature=%r, TopK=%r, TopP=%r, MinP=%r, RepeatPenalty=%r, "
                "RepeatWindow=%r, Seed=%r)" % (self.Temperature, self.TopK, self.TopP, self.MinP,
                                               self.RepeatPenalty, self.RepeatWindow, self.Seed))


class _Outputs(C.Structure):
    _fields_ = [
        ("tokens", C.c_void_p),
        ("topk_idx", C.c_void_p),
        ("topk_prob", C.c_void_p),
        ("topk_stride", C.c_int32),
        ("flags", C.c_void_p),
        ("uniforms", C.c_void_p),
    ]


class _GGUFInfo(C.Structure):
    _fields_ = [
        ("version", C.c_uint32),
        ("alignment", C.c_uint32),
        ("tensor_count", C.c_uint64),
        ("metadata_count", C.c_uint64),
        ("file_size", C.c_uint64),
        ("data_offset", C.c_uint64),
    ]


class _GGUFTensor(C.Structure):
    _fields_ = [
        ("type", C.c_int32),
        ("n_dims", C.c_int32),
        ("dims", C.c_uint64 * 4),
        ("nbytes", C.c_uint64),
        ("file_offset", C.c_uint64),
        ("data", C.c_void_p),
    ]


_lib = None

# Every entry point declared in include/vdx_sampler.h, with its ctypes signature.
_SIGNATURES = {
    "vdx_sampler_default_config": (None, [C.POINTER(TVdxSamplerConfig)]),
    "vdx_sampler_create": (C.c_int, [C.POINTER(C.c_void_p), C.c_int32, C.c_int32]),
    "vdx_sampler_destroy": (None, [C.c_void_p]),
    "vdx_sampler_set_config": (C.c_int, [C.c_void_p, C.POINTER(TVdxSamplerConfig)]),
    "vdx_sampler_get_config": (C.c_int, [C.c_void_p, C.POINTER(TVdxSamplerConfig)]),
    "vdx_sampler_set_row_config": (C.c_int, [C.c_void_p, C.c_int32, C.POINTER(TVdxSamplerConfig)]),
    "vdx_sampler_get_row_config": (C.c_int, [C.c_void_p, C.c_int32, C.POINTER(TVdxSamplerConfig)]),
    "vdx_sampler_save_row_state": (C.c_int64, [C.c_void_p, C.c_int32, C.c_void_p, C.c_int64]),
    "vdx_sampler_load_row_state": (C.c_int, [C.c_void_p, C.c_int32, C.c_void_p, C.c_int64]),
    "vdx_sampler_process": (C.c_int32, [C.c_void_p, C.POINTER(C.c_float), C.c_int32]),
    "vdx_sampler_process_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                             C.c_int64, C.c_void_p, C.POINTER(_Outputs),
                                             C.c_void_p]),
    "vdx_sample_device_noalloc": (C.c_int, [C.POINTER(TVdxSamplerConfig), C.c_void_p, C.c_int32, C.c_int32,
                                            C.c_int64, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p,
                                            C.POINTER(_Outputs), C.c_void_p]),
    "vdx_lmhead_q4_0": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_int32,
                                  C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p]),
    "vdx_lmhead": (C.c_int, [C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p, C.c_float, C.c_int32,
                             C.c_int32, C.c_int32, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p]),
    "vdx_lmhead_packed_bytes": (C.c_int64, [C.c_int32, C.c_int32, C.c_int32]),
    "vdx_lmhead_pack": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_void_p, C.c_int64,
                                  C.c_void_p]),
    "vdx_sampler_lmhead_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p,
                                            C.c_float, C.c_int32, C.c_int32, C.c_int32, C.c_void_p,
                                            C.c_int64, C.c_void_p, C.POINTER(_Outputs), C.c_void_p]),
    "vdx_sampler_lmhead_q4_0_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32,
                                                 C.c_int32, C.c_int32, C.c_void_p, C.c_int64,
                                                 C.c_void_p, C.POINTER(_Outputs), C.c_void_p]),
    "vdx_sampler_add_to_history": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32]),
    "vdx_sampler_add_to_history_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32,
                                                    C.c_void_p]),
    "vdx_sampler_reset_history": (C.c_int, [C.c_void_p, C.c_int32]),
    "vdx_sampler_set_history": (C.c_int, [C.c_void_p, C.c_int32, C.POINTER(C.c_int32), C.c_int32,
                                          C.c_int32]),
    "vdx_sampler_get_history": (C.c_int32, [C.c_void_p, C.c_int32, C.POINTER(C.c_int32),
                                            C.c_int32, C.POINTER(C.c_int32)]),
    "vdx_sampler_set_rng": (C.c_int, [C.c_void_p, C.c_int32]),
    "vdx_sampler_set_timing": (C.c_int, [C.c_void_p, C.c_int32]),
    "vdx_sampler_get_timing": (C.c_int, [C.c_void_p, C.c_int32, C.POINTER(C.c_double),
                                         C.POINTER(C.c_int64)]),
    "vdx_gguf_open": (C.c_int, [C.POINTER(C.c_void_p), C.c_char_p]),
    "vdx_gguf_close": (None, [C.c_void_p]),
    "vdx_gguf_last_error": (C.c_char_p, [C.c_void_p]),
    "vdx_gguf_get_info": (C.c_int, [C.c_void_p, C.POINTER(_GGUFInfo)]),
    "vdx_gguf_tensor_name": (C.c_int, [C.c_void_p, C.c_int64, C.c_char_p, C.c_int32]),
    "vdx_gguf_find_tensor": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(_GGUFTensor)]),
    "vdx_gguf_meta_key": (C.c_int, [C.c_void_p, C.c_int64, C.c_char_p, C.c_int32]),
    "vdx_gguf_meta_type": (C.c_int, [C.c_void_p, C.c_char_p]),
    "vdx_gguf_meta_int": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_int64)]),
    "vdx_gguf_meta_float": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_double)]),
    "vdx_gguf_meta_string": (C.c_int, [C.c_void_p, C.c_char_p, C.c_char_p, C.c_int32]),
    "vdx_gguf_meta_array": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_int32),
                                      C.POINTER(C.c_int64)]),
    "vdx_sampler_last_error": (C.c_char_p, [C.c_void_p]),
    "vdx_sampler_version": (C.c_char_p, []),
}


def lib_path() -> str:
    return _build.LIB


def load_library():
    """Loads libvdxsampler.so (built by vindexllm_amd.build); raises if absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(_build.LIB):
            raise RuntimeError(f"{_build.LIB} is not built; run __graft_entry__.build()")
        # One HIP runtime per process: where PyTorch is installed, its bundled
        # libamdhip64 is loaded first, so the library binds to the same one
        # (loading ROCm's first leaves torch's devices unavailable).
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(_build.LIB)
        for name, (res, args) in _SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _err(s) -> str:
    m = load_library().vdx_sampler_last_error(s)
    return m.decode() if m else ""


class TVdxSampler:
    """TVdxSampler (Sampler.pas:37-91) backed by the GPU library.

    ``max_rows`` is the largest batch ``process_device`` will be given; the
    host-pointer ``Process`` samples row 0.
    """

    def __init__(self, device: int = 0, max_rows: int = 1):
        L = load_library()
        h = C.c_void_p()
        rc = L.vdx_sampler_create(C.byref(h), int(device), int(max_rows))
        if rc != VDX_OK:
            raise VdxSamplerError(rc, _err(None))
        self._h = h
        self.max_rows = int(max_rows)
        self.device = int(device)
        self._errors = []

    # -- lifetime ---------------------------------------------------------
    def Free(self):
        if getattr(self, "_h", None):
            load_library().vdx_sampler_destroy(self._h)
            self._h = None

    close = Free

    def __del__(self):
        try:
            self.Free()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.Free()

    def _check(self, rc: int) -> int:
        if rc < 0:
            msg = _err(self._h)
            self._errors.append(msg)
            raise VdxSamplerError(rc, msg)
        return rc

    def GetErrors(self):
        """Messages of failed calls (the reference keeps a TVdxErrors list)."""
        return list(self._errors)

    # -- configuration (Sampler.pas:100-155) --------------------------------
    @staticmethod
    def DefaultConfig() -> TVdxSamplerConfig:
        c = TVdxSamplerConfig()
        load_library().vdx_sampler_default_config(C.byref(c))
        return c

    def SetConfig(self, cfg: TVdxSamplerConfig):
        self._check(load_library().vdx_sampler_set_config(self._h, C.byref(cfg)))

    def GetConfig(self) -> TVdxSamplerConfig:
        c = TVdxSamplerConfig()
        self._check(load_library().vdx_sampler_get_config(self._h, C.byref(c)))
        return c

    def SetRng(self, kind: int):
        self._check(load_library().vdx_sampler_set_rng(self._h, int(kind)))

    # -- per-row configs and checkpoints (beyond the reference) -------------
    def SetRowConfig(self, row: int, cfg: TVdxSamplerConfig):
        """SetConfig for one row of the batch (SetConfig's rules applied to
        that row; a changed Seed reseeds the row from Seed itself, so the row
        draws what a reference sampler with ``cfg`` draws)."""
        self._check(load_library().vdx_sampler_set_row_config(self._h, int(row), C.byref(cfg)))

    def GetRowConfig(self, row: int) -> TVdxSamplerConfig:
        c = TVdxSamplerConfig()
        self._check(load_library().vdx_sampler_get_row_config(self._h, int(row), C.byref(c)))
        return c

    def save_row_state(self, row: int) -> bytes:
        """The row's sampler state (config, RNG state, history ring) as bytes."""
        L = load_library()
        n = self._check(L.vdx_sampler_save_row_state(self._h, int(row), None, 0))
        buf = C.create_string_buffer(n)
        self._check(L.vdx_sampler_save_row_state(self._h, int(row), buf, n))
        return buf.raw

    def load_row_state(self, row: int, blob: bytes):
        b = bytes(blob)
        self._check(load_library().vdx_sampler_load_row_state(self._h, int(row), b, len(b)))

    def save_state(self):
        """Every row's state (a list of blobs, row order)."""
        return [self.save_row_state(r) for r in range(self.max_rows)]

    def load_state(self, blobs):
        for r, b in enumerate(blobs):
            self.load_row_state(r, b)

    # -- sampling -------------------------------------------------------------
    def Process(self, logits, vocab_size: int | None = None) -> int:
        """Process (Sampler.pas:265-528) on a host float32 numpy array, which is
        penalised in place as in the reference; returns the token id."""
        import numpy as np

        assert isinstance(logits, np.ndarray) and logits.dtype == np.float32
        assert logits.flags["C_CONTIGUOUS"]
        V = int(logits.shape[-1] if vocab_size is None else vocab_size)
        ptr = logits.ctypes.data_as(C.POINTER(C.c_float))
        return self._check(load_library().vdx_sampler_process(self._h, ptr, V))

    def process_device(self, logits, uniforms=None, tokens=None, topk_idx=None, topk_prob=None,
                       flags=None, uniforms_out=None, rows: int | None = None,
                       vocab: int | None = None, row_stride: int | None = None, stream=None):
        """Samples ``rows`` device-resident rows of ``logits`` (a float32 GPU
        tensor, row r at offset r*row_stride; penalised in place).
        ``uniforms`` (float32 GPU tensor, one per row) replaces the RNG draw.
        Returns the int32 token tensor; asynchronous on ``stream`` (default:
        torch's current stream)."""
        import torch

        assert logits.is_cuda and logits.dtype == torch.float32
        if logits.dim() == 1:
            logits = logits.view(1, -1)
        B = int(logits.shape[0] if rows is None else rows)
        V = int(logits.shape[-1] if vocab is None else vocab)
        stride = int(logits.stride(0) if row_stride is None else row_stride)
        if tokens is None:
            tokens = torch.empty(B, dtype=torch.int32, device=logits.device)
        o = _Outputs()
        o.tokens = tokens.data_ptr()
        o.topk_idx = topk_idx.data_ptr() if topk_idx is not None else None
        o.topk_prob = topk_prob.data_ptr() if topk_prob is not None else None
        o.topk_stride = int(topk_idx.shape[-1] if topk_idx is not None else
                            (topk_prob.shape[-1] if topk_prob is not None else 0))
        o.flags = flags.data_ptr() if flags is not None else None
        o.uniforms = uniforms_out.data_ptr() if uniforms_out is not None else None
        if uniforms is not None:
            assert uniforms.is_cuda and uniforms.dtype == torch.float32 and uniforms.numel() >= B
        st = stream if stream is not None else torch.cuda.current_stream(logits.device)
        self._check(load_library().vdx_sampler_process_device(
            self._h, C.c_void_p(logits.data_ptr()), B, V, stride,
            C.c_void_p(uniforms.data_ptr()) if uniforms is not None else None, C.byref(o),
            C.c_void_p(st.cuda_stream)))
        return tokens

    def lmhead_device(self, weights, wtype: int, hidden, vocab: int, norm_weight=None,
                      norm_eps: float = 1e-6, logits=None, uniforms=None, tokens=None,
                      topk_idx=None, topk_prob=None, flags=None, uniforms_out=None, stream=None):
        """RunUnembedding + Process (Inference.pas:327-339) on the GPU: the output
        RMSNorm (``norm_weight``, float32 GPU tensor of in_dim; None skips it)
        and the lm_head in ``wtype`` (VDX_TENSOR_Q4_0 / _Q8_0 / _F16; ``weights``:
        uint8 GPU tensor, vocab rows in that GGUF layout) over ``hidden`` (rows x
        in_dim float32 GPU tensor) write logits into ``logits`` (rows x >= vocab
        float32 GPU tensor) or the sampler's workspace, and the rows are sampled
        as by ``process_device``."""
        import torch

        assert hidden.is_cuda and hidden.dtype == torch.float32 and hidden.is_contiguous()
        assert weights.is_cuda and weights.dtype == torch.uint8
        if hidden.dim() == 1:
            hidden = hidden.view(1, -1)
        B, D = int(hidden.shape[0]), int(hidden.shape[1])
        if tokens is None:
            tokens = torch.empty(B, dtype=torch.int32, device=hidden.device)
        o = _Outputs()
        o.tokens = tokens.data_ptr()
        o.topk_idx = topk_idx.data_ptr() if topk_idx is not None else None
        o.topk_prob = topk_prob.data_ptr() if topk_prob is not None else None
        o.topk_stride = int(topk_idx.shape[-1] if topk_idx is not None else
                            (topk_prob.shape[-1] if topk_prob is not None else 0))
        o.flags = flags.data_ptr() if flags is not None else None
        o.uniforms = uniforms_out.data_ptr() if uniforms_out is not None else None
        lp, ls = None, 0
        if logits is not None:
            assert logits.is_cuda and logits.dtype == torch.float32
            lp, ls = C.c_void_p(logits.data_ptr()), int(logits.stride(0))
        nw = None
        if norm_weight is not None:
            assert norm_weight.is_cuda and norm_weight.dtype == torch.float32 and norm_weight.numel() >= D
            nw = C.c_void_p(norm_weight.data_ptr())
        st = stream if stream is not None else torch.cuda.current_stream(hidden.device)
        self._check(load_library().vdx_sampler_lmhead_device(
            self._h, C.c_void_p(weights.data_ptr()), int(wtype), C.c_void_p(hidden.data_ptr()), nw,
            float(norm_eps), B, D, int(vocab), lp, ls,
            C.c_void_p(uniforms.data_ptr()) if uniforms is not None else None, C.byref(o),
            C.c_void_p(st.cuda_stream)))
        return tokens

    def lmhead_q4_0_device(self, weights, hidden, vocab: int, logits=None, uniforms=None,
                           tokens=None, topk_idx=None, topk_prob=None, flags=None,
                           uniforms_out=None, stream=None):
        """lmhead_device for a Q4_0 head without the output norm."""
        return self.lmhead_device(weights, VDX_TENSOR_Q4_0, hidden, vocab, logits=logits,
                                  uniforms=uniforms, tokens=tokens, topk_idx=topk_idx,
                                  topk_prob=topk_prob, flags=flags, uniforms_out=uniforms_out,
                                  stream=stream)

    def set_timing(self, enable: bool):
        self._check(load_library().vdx_sampler_set_timing(self._h, 1 if enable else 0))

    def get_timing(self, which: int = 0):
        """(total_ms, count) of the event-timed sampling kernels (which=0),
        penalty kernels (1) or whole calls (2) since the last query."""
        t = C.c_double()
        n = C.c_int64()
        self._check(load_library().vdx_sampler_get_timing(self._h, int(which), C.byref(t),
                                                           C.byref(n)))
        return t.value, n.value

    # -- history (Sampler.pas:530-549) ----------------------------------------
    def AddToHistory(self, token_id: int, row: int = 0):
        self._check(load_library().vdx_sampler_add_to_history(self._h, int(row), int(token_id)))

    def add_to_history_device(self, tokens, stream=None):
        import torch

        st = stream if stream is not None else torch.cuda.current_stream(tokens.device)
        self._check(load_library().vdx_sampler_add_to_history_device(
            self._h, C.c_void_p(tokens.data_ptr()), int(tokens.numel()), C.c_void_p(st.cuda_stream)))

    def ResetHistory(self, row: int = -1):
        self._check(load_library().vdx_sampler_reset_history(self._h, int(row)))

    def set_history(self, row: int, ids, pos: int | None = None):
        import numpy as np

        a = np.ascontiguousarray(ids, dtype=np.int32)
        n = int(a.size)
        p = (n % max(self.GetRowConfig(row).RepeatWindow, 1)) if pos is None else int(pos)
        self._check(load_library().vdx_sampler_set_history(
            self._h, int(row), a.ctypes.data_as(C.POINTER(C.c_int32)) if n else None, n, p))

    def get_history(self, row: int = 0):
        import numpy as np

        cap = max(self.GetRowConfig(row).RepeatWindow, 0)
        buf = np.zeros(max(cap, 1), dtype=np.int32)
        pos = C.c_int32()
        n = self._check(load_library().vdx_sampler_get_history(
            self._h, int(row), buf.ctypes.data_as(C.POINTER(C.c_int32)), cap, C.byref(pos)))
        return buf[:n].tolist(), pos.value


def lmhead(weights, wtype: int, hidden, vocab: int, norm_weight=None, norm_eps: float = 1e-6,
           logits=None, scratch=None, stream=None):
    """UnembedToLogits alone (Model.pas:1258-1270): the optional output RMSNorm
    then the lm_head in ``wtype`` (VDX_TENSOR_Q4_0 / _Q8_0 / _F16), batched over
    the rows of ``hidden``; returns the rows x vocab float32 logits tensor (or
    fills ``logits``).  ``scratch`` (float32 GPU tensor of >= 16*in_dim) is
    allocated here when needed and not given."""
    import torch

    assert hidden.is_cuda and hidden.dtype == torch.float32 and hidden.is_contiguous()
    assert weights.is_cuda and weights.dtype == torch.uint8
    if hidden.dim() == 1:
        hidden = hidden.view(1, -1)
    B, D = int(hidden.shape[0]), int(hidden.shape[1])
    if logits is None:
        logits = torch.empty(B, int(vocab), dtype=torch.float32, device=hidden.device)
    if scratch is None and (B > 1 or norm_weight is not None):
        scratch = torch.empty(16 * D, dtype=torch.float32, device=hidden.device)
    nw = None
    if norm_weight is not None:
        assert norm_weight.is_cuda and norm_weight.dtype == torch.float32 and norm_weight.numel() >= D
        nw = C.c_void_p(norm_weight.data_ptr())
    st = stream if stream is not None else torch.cuda.current_stream(hidden.device)
    rc = load_library().vdx_lmhead(C.c_void_p(weights.data_ptr()), int(wtype),
                                   C.c_void_p(hidden.data_ptr()), nw, float(norm_eps), B, D,
                                   int(vocab), C.c_void_p(logits.data_ptr()), int(logits.stride(0)),
                                   C.c_void_p(scratch.data_ptr()) if scratch is not None else None,
                                   C.c_void_p(st.cuda_stream))
    if rc != VDX_OK:
        raise VdxSamplerError(rc, _err(None))
    return logits


def lmhead_packed_bytes(wtype: int, in_dim: int, vocab: int) -> int:
    n = load_library().vdx_lmhead_packed_bytes(int(wtype), int(in_dim), int(vocab))
    if n < 0:
        raise VdxSamplerError(int(n), "lm_head pack: need a VDX_TENSOR_* format and in_dim % 32 == 0")
    return int(n)


def lmhead_pack(weights, wtype: int, in_dim: int, vocab: int, out=None, stream=None):
    """The lm_head weights (uint8 GPU tensor in the GGUF layout of ``wtype``)
    repacked once for coalesced, line-aligned loads; pass the result with
    ``wtype | VDX_LMHEAD_PACKED`` to ``lmhead`` / ``TVdxSampler.lmhead_device``
    (bit-identical logits)."""
    import torch

    assert weights.is_cuda and weights.dtype == torch.uint8
    n = lmhead_packed_bytes(wtype, in_dim, vocab)
    if out is None:
        out = torch.empty(n, dtype=torch.uint8, device=weights.device)
    st = stream if stream is not None else torch.cuda.current_stream(weights.device)
    rc = load_library().vdx_lmhead_pack(C.c_void_p(weights.data_ptr()), int(wtype), int(in_dim), int(vocab),
                                        C.c_void_p(out.data_ptr()), int(out.numel()), C.c_void_p(st.cuda_stream))
    if rc != VDX_OK:
        raise VdxSamplerError(rc, _err(None))
    return out


def lmhead_q4_0(weights, hidden, vocab: int, logits=None, scratch=None, stream=None):
    """The Q4_0 lm_head alone (matvec_q4_0.comp, batched), without the norm."""
    return lmhead(weights, VDX_TENSOR_Q4_0, hidden, vocab, logits=logits, scratch=scratch, stream=stream)


def sample_device_noalloc(cfg: TVdxSamplerConfig, logits, uniforms, history=None, history_count=None,
                          tokens=None, topk_idx=None, topk_prob=None, flags=None, uniforms_out=None,
                          rows: int | None = None, vocab: int | None = None, row_stride: int | None = None,
                          stream=None):
    """vdx_sample_device_noalloc: samples device-resident rows with the
    library's fixed workspace (no sampler object, nothing allocated by the
    library).  ``uniforms`` (float32 GPU tensor, one per row) is required;
    ``history`` (int32 GPU tensor, rows x stride) with ``history_count``
    (int32 GPU tensor, one per row) gives each row's ring for the penalty.
    Returns the int32 token tensor (``tokens`` when given)."""
    import torch

    assert logits.is_cuda and logits.dtype == torch.float32
    if logits.dim() == 1:
        logits = logits.view(1, -1)
    B = int(logits.shape[0] if rows is None else rows)
    V = int(logits.shape[-1] if vocab is None else vocab)
    stride = int(logits.stride(0) if row_stride is None else row_stride)
    assert uniforms.is_cuda and uniforms.dtype == torch.float32 and uniforms.numel() >= B
    if tokens is None:
        tokens = torch.empty(B, dtype=torch.int32, device=logits.device)
    o = _Outputs()
    o.tokens = tokens.data_ptr()
    o.topk_idx = topk_idx.data_ptr() if topk_idx is not None else None
    o.topk_prob = topk_prob.data_ptr() if topk_prob is not None else None
    o.topk_stride = int(topk_idx.shape[-1] if topk_idx is not None else
                        (topk_prob.shape[-1] if topk_prob is not None else 0))
    o.flags = flags.data_ptr() if flags is not None else None
    o.uniforms = uniforms_out.data_ptr() if uniforms_out is not None else None
    hs = 0
    if history is not None:
        assert history.is_cuda and history.dtype == torch.int32 and history.dim() == 2
        assert history_count is not None and history_count.dtype == torch.int32
        hs = int(history.stride(0))
    st = stream if stream is not None else torch.cuda.current_stream(logits.device)
    rc = load_library().vdx_sample_device_noalloc(
        C.byref(cfg), C.c_void_p(logits.data_ptr()), B, V, stride, C.c_void_p(uniforms.data_ptr()),
        C.c_void_p(history.data_ptr()) if history is not None else None, hs,
        C.c_void_p(history_count.data_ptr()) if history is not None else None, C.byref(o),
        C.c_void_p(st.cuda_stream))
    if rc < 0:
        raise VdxSamplerError(rc, _err(None))
    return tokens


def version() -> str:
    return load_library().vdx_sampler_version().decode()
