"""Python host binding of the gfx950 token sampler (libgs_sampler.so).

Mirrors the reference interface of gguf-rs-cli's src/sampler.rs:

    set_seed(s)                                          src/sampler.rs:5
    sample(logits, temperature, top_k, top_p,
           rep_penalty, recent) -> int                   src/sampler.rs:35-36

with the same argument meaning, the same process-global LCG stream
(one draw per call iff temperature > 0) and errors where the reference
panics (NaN logits, empty logits with T > 0).  It adds the `Sampler`
object (construction = params + seed) and a batched entry over B rows of
device-resident logits.

The library must be built (gguf-rs-cli_amd/build.py).  There is no CPU
fallback: if the HIP library is missing, importing this module fails.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgs_sampler.so")

GS_OK = 0
GS_ERR_INVALID = -1
GS_ERR_EMPTY = -2
GS_ERR_NAN = -3
GS_ERR_HIP = -5
GS_ERR_NOMEM = -6
GS_ERR_UNSUPPORTED = -7
_ERRNAMES = {
    GS_ERR_INVALID: "invalid argument",
    GS_ERR_EMPTY: "empty logits (reference panics at pairs[0], src/sampler.rs:53)",
    GS_ERR_NAN: "NaN logit (reference panics in partial_cmp().unwrap(), src/sampler.rs:17,45)",
    GS_ERR_HIP: "HIP runtime error",
    GS_ERR_NOMEM: "device allocation failed",
    GS_ERR_UNSUPPORTED: "outside implemented limits",
}

# Symbols declared in include/gs_sampler.h.
EXPORTS = [
    "gs_sampler_create", "gs_sampler_destroy", "gs_sampler_set_params",
    "gs_sampler_set_seed", "gs_sampler_get_state", "gs_sampler_set_state",
    "gs_sampler_reserve", "gs_sample", "gs_sample_mut", "gs_logits_writeback", "gs_sample_detail", "gs_sample_batch", "gs_sample_batch_noalloc", "gs_window_push",
    "gs_synth_logits", "gs_limits", "gs_version",
    # include/gs_gemv.h
    "gs_qmatrix_upload", "gs_qmatrix_destroy", "gs_qmatrix_shape", "gs_gemv",
    # include/gs_decode.h
    "gs_sampler_get_params", "gs_sampler_fallback_rows", "gs_decode_init", "gs_decode_commit", "gs_decode_step",
    # include/gs_tokens.h
    "gs_vocab_create", "gs_vocab_destroy", "gs_vocab_find", "gs_token_decode", "gs_tokens_decode",
    "gs_chat_template_detect", "gs_stop_tokens",
]


class SamplerError(RuntimeError):
    def __init__(self, code, where=""):
        self.code = code
        super().__init__("%s: %s (%d)" % (where or "gs_sampler", _ERRNAMES.get(code, "error"), code))


class GsParams(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_uint32),
                ("top_p", ctypes.c_float), ("rep_penalty", ctypes.c_float)]


class GsDetail(ctypes.Structure):
    """gs_detail (include/gs_sampler.h)."""
    _fields_ = [("ids", ctypes.c_void_p), ("p", ctypes.c_void_p), ("cap", ctypes.c_size_t),
                ("n_kept", ctypes.c_void_p), ("cut", ctypes.c_void_p), ("sums", ctypes.c_void_p),
                ("ties", ctypes.c_void_p)]


class DecodeCtx(ctypes.Structure):
    """gs_decode_ctx (include/gs_decode.h)."""
    _fields_ = [("B", ctypes.c_size_t), ("rows", ctypes.c_void_p), ("window", ctypes.c_void_p),
                ("ld_window", ctypes.c_size_t), ("W", ctypes.c_size_t), ("window_len", ctypes.c_void_p),
                ("stop", ctypes.c_void_p), ("n_stop", ctypes.c_size_t), ("max_new", ctypes.c_uint32),
                ("generated", ctypes.c_void_p), ("ld_generated", ctypes.c_size_t), ("next", ctypes.c_void_p),
                ("u", ctypes.c_void_p), ("tokens", ctypes.c_void_p), ("status", ctypes.c_void_p),
                ("n_active", ctypes.c_void_p)]


_lib = None


def load_library(path=LIB_PATH):
    """Load libgs_sampler.so (raises OSError if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise OSError("libgs_sampler.so not built: run gguf-rs-cli_amd/build.py (%s)" % path)
    lib = ctypes.CDLL(path)
    P, U64, SZ, I = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_size_t, ctypes.c_int
    sig = {
        "gs_sampler_create": ([ctypes.POINTER(GsParams), U64, ctypes.POINTER(P)], I),
        "gs_sampler_destroy": ([P], I),
        "gs_sampler_set_params": ([P, ctypes.POINTER(GsParams)], I),
        "gs_sampler_set_seed": ([P, U64], I),
        "gs_sampler_get_state": ([P, ctypes.POINTER(U64)], I),
        "gs_sampler_set_state": ([P, U64], I),
        "gs_sampler_reserve": ([P, SZ, SZ], I),
        "gs_sample": ([P, P, SZ, P, SZ, ctypes.POINTER(ctypes.c_uint32)], I),
        "gs_sample_mut": ([P, P, SZ, P, SZ, ctypes.POINTER(ctypes.c_uint32)], I),
        "gs_logits_writeback": ([P, P, SZ, SZ, SZ, P, P, SZ, P, SZ, P], I),
        "gs_sample_detail": ([P, P, SZ, SZ, SZ, P, P, SZ, P, SZ, P, P, P, ctypes.POINTER(GsDetail), P], I),
        "gs_sample_batch": ([P, P, SZ, SZ, SZ, P, P, SZ, P, SZ, P, P, P, P], I),
        "gs_sample_batch_noalloc": ([P, P, SZ, SZ, SZ, P, P, SZ, P, SZ, P, P, P, P], I),
        "gs_window_push": ([P, SZ, SZ, SZ, SZ, P, P], I),
        "gs_synth_logits": ([P, SZ, SZ, SZ, U64, U64, ctypes.c_float, P], I),
        "gs_limits": ([ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32)], I),
        "gs_version": ([], ctypes.c_char_p),
        "gs_qmatrix_upload": ([ctypes.c_uint32, P, SZ, SZ, ctypes.POINTER(P)], I),
        "gs_qmatrix_destroy": ([P], I),
        "gs_qmatrix_shape": ([P, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(SZ), ctypes.POINTER(SZ)], I),
        "gs_gemv": ([P, P, SZ, P, P], I),
        "gs_sampler_get_params": ([P, ctypes.POINTER(GsParams)], I),
        "gs_sampler_fallback_rows": ([P, P, ctypes.POINTER(ctypes.c_size_t)], I),
        "gs_decode_init": ([P, P, ctypes.POINTER(DecodeCtx), P, P, P], I),
        "gs_decode_commit": ([P, P, ctypes.POINTER(DecodeCtx), P], I),
        "gs_decode_step": ([P, P, P, P, SZ, SZ, P, ctypes.POINTER(DecodeCtx), P], I),
        "gs_vocab_create": ([P, P, SZ, P, SZ, ctypes.c_uint32, ctypes.POINTER(P)], I),
        "gs_vocab_destroy": ([P], I),
        "gs_vocab_find": ([P, ctypes.c_char_p, SZ, ctypes.POINTER(ctypes.c_uint32)], I),
        "gs_token_decode": ([P, ctypes.c_uint32, P, SZ, ctypes.POINTER(SZ)], I),
        "gs_tokens_decode": ([P, P, SZ, P, SZ, ctypes.POINTER(SZ)], I),
        "gs_chat_template_detect": ([P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)], I),
        "gs_stop_tokens": ([P, ctypes.c_uint32, P, SZ, P, SZ, ctypes.POINTER(SZ)], I),
    }
    for name, (args, res) in sig.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = res
    _lib = lib
    return lib


def _check(rc, where):
    if rc != GS_OK:
        raise SamplerError(rc, where)


def _ptr(x):
    """Device/host address of a torch tensor, numpy array, int or None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if hasattr(x, "ctypes"):
        return x.ctypes.data
    raise TypeError("unsupported buffer type %r" % type(x))


_TORCH = None


def _torch_fast_args(logits, recent):
    """(ptr, V, recent ptr, W) for a contiguous torch f32 row and a window
    that is a torch tensor of 4-byte ids, a contiguous numpy uint32 array or
    None / empty; None for anything else."""
    global _TORCH
    if _TORCH is None:
        import sys
        t = sys.modules.get("torch")
        if t is None:
            return None
        import numpy as np
        _TORCH = (t.Tensor, t.float32, (t.int32, t.uint32), np.ndarray, np.dtype(np.uint32))
    tensor, f32, ids, ndarray, u32 = _TORCH
    if type(logits) is not tensor or logits.dtype is not f32 or not logits.is_contiguous():
        return None
    if recent is None or (type(recent) is tuple and not recent):
        return logits.data_ptr(), logits.numel(), None, 0
    if type(recent) is ndarray:
        if recent.dtype != u32 or not recent.flags.c_contiguous:
            return None
        W = recent.size
        return logits.data_ptr(), logits.numel(), (recent.ctypes.data if W else None), W
    if type(recent) is not tensor or recent.dtype not in ids or not recent.is_contiguous():
        return None
    W = recent.numel()
    return logits.data_ptr(), logits.numel(), (recent.data_ptr() if W else None), W


def _stream_handle(stream):
    """The HIP stream of a call: `stream` (a torch.cuda.Stream or a handle),
    or by default torch's current stream when torch has initialised the GPU
    (so calls order with torch's work, inside torch.cuda.stream() blocks and
    under graph capture), else the NULL stream."""
    if stream is None:
        import sys as _sys
        torch = _sys.modules.get("torch")
        if torch is not None and torch.cuda.is_initialized():
            return torch.cuda.current_stream().cuda_stream
        return None
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream  # torch.cuda.Stream


class Sampler:
    """Sampler construction of the drop-in: the four scalars of
    src/sampler.rs:35-36 plus the LCG seed of src/sampler.rs:3-5.
    Defaults are the reference CLI's (src/main.rs:24-31, 48-49)."""

    def __init__(self, temperature=0.7, top_k=40, top_p=0.9, rep_penalty=1.1, seed=42):
        self._lib = load_library()
        self._h = ctypes.c_void_p()
        self.params = GsParams(temperature, top_k, top_p, rep_penalty)
        self._out = ctypes.c_uint32()
        self._outref = ctypes.byref(self._out)
        _check(self._lib.gs_sampler_create(ctypes.byref(self.params), seed, ctypes.byref(self._h)),
               "gs_sampler_create")

    def close(self):
        if self._h:
            self._lib.gs_sampler_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_params(self, temperature, top_k, top_p, rep_penalty):
        self.params = GsParams(temperature, top_k, top_p, rep_penalty)
        _check(self._lib.gs_sampler_set_params(self._h, ctypes.byref(self.params)), "set_params")

    def fallback_rows(self, stream=None):
        """Rows of the last full-vocabulary call finished by the fallback
        forms instead of the increment-histogram path (waits for the stream)."""
        n = ctypes.c_size_t()
        _check(self._lib.gs_sampler_fallback_rows(self._h, _stream_handle(stream), ctypes.byref(n)), "fallback_rows")
        return n.value

    def set_seed(self, seed):
        _check(self._lib.gs_sampler_set_seed(self._h, seed), "set_seed")

    @property
    def state(self):
        v = ctypes.c_uint64()
        _check(self._lib.gs_sampler_get_state(self._h, ctypes.byref(v)), "get_state")
        return v.value

    @state.setter
    def state(self, v):
        _check(self._lib.gs_sampler_set_state(self._h, v), "set_state")

    def reserve(self, B, V):
        _check(self._lib.gs_sampler_reserve(self._h, B, V), "reserve")

    def sample(self, logits, recent=()):
        """sample(logits, recent) -> token; logits: numpy f32 (host) or a
        torch f32 tensor (host or device).  Synchronous."""
        fast = _torch_fast_args(logits, recent)
        if fast is not None:
            if logits.is_cuda or (recent is not None and getattr(recent, "is_cuda", False)):
                # gs_sample runs on the sampler's own non-blocking stream:
                # wait for torch's current stream, which may still be writing
                # the logits (or the window)
                import torch
                torch.cuda.current_stream(logits.device if logits.is_cuda else None).synchronize()
            rc = self._lib.gs_sample(self._h, fast[0], fast[1], fast[2], fast[3], self._outref)
            if rc != GS_OK:
                raise SamplerError(rc, "gs_sample")
            return self._out.value
        import numpy as np
        keep = []
        if isinstance(logits, (list, tuple)):
            logits = np.asarray(logits, dtype=np.float32)
        if hasattr(logits, "dtype") and str(logits.dtype) not in ("float32", "torch.float32"):
            raise TypeError("logits must be float32")
        if hasattr(logits, "is_contiguous") and not logits.is_contiguous():
            raise TypeError("logits must be contiguous")
        if isinstance(logits, np.ndarray):
            logits = np.ascontiguousarray(logits)
            keep.append(logits)
        V = int(logits.numel() if hasattr(logits, "numel") else logits.size)
        if recent is None or (not hasattr(recent, "data_ptr") and not hasattr(recent, "ctypes")):
            recent = np.ascontiguousarray(np.asarray(list(recent or ()), dtype=np.uint32))
        elif isinstance(recent, np.ndarray):
            recent = np.ascontiguousarray(recent.astype(np.uint32, copy=False))   # ids are u32 (&[u32])
        keep.append(recent)
        if hasattr(recent, "element_size") and recent.element_size() != 4:
            raise TypeError("recent ids must be 4-byte integers")
        W = int(recent.numel() if hasattr(recent, "numel") else recent.size)
        out = ctypes.c_uint32()
        _check(self._lib.gs_sample(self._h, _ptr(logits), V, _ptr(recent) if W else None, W,
                                   ctypes.byref(out)), "gs_sample")
        return int(out.value)

    def sample_mut(self, logits, recent=()):
        """sample(&mut logits, ...) as the reference takes it: returns the
        token and leaves `logits` (a contiguous numpy f32 array, or a torch
        f32 tensor on the host or the device) penalized and divided by T
        (src/sampler.rs:37,41), in place."""
        import numpy as np
        if isinstance(logits, np.ndarray):
            if logits.dtype != np.float32 or not logits.flags.c_contiguous or not logits.flags.writeable:
                raise TypeError("logits must be a writeable contiguous float32 array")
        elif hasattr(logits, "data_ptr"):
            if str(logits.dtype) != "torch.float32" or not logits.is_contiguous():
                raise TypeError("logits must be a contiguous float32 tensor")
            if logits.is_cuda:
                import torch
                torch.cuda.current_stream(logits.device).synchronize()
        else:
            raise TypeError("logits must be a numpy array or a torch tensor (mutated in place)")
        V = int(logits.numel() if hasattr(logits, "numel") else logits.size)
        if recent is None or (not hasattr(recent, "data_ptr") and not hasattr(recent, "ctypes")):
            recent = np.ascontiguousarray(np.asarray(list(recent or ()), dtype=np.uint32))
        elif isinstance(recent, np.ndarray):
            recent = np.ascontiguousarray(recent.astype(np.uint32, copy=False))
        W = int(recent.numel() if hasattr(recent, "numel") else recent.size)
        out = ctypes.c_uint32()
        _check(self._lib.gs_sample_mut(self._h, _ptr(logits), V, _ptr(recent) if W else None, W,
                                       ctypes.byref(out)), "gs_sample_mut")
        return int(out.value)

    def logits_writeback(self, logits, params=None, recent=None, recent_len=None, stream=None,
                         V=None, ld=None, W=None, ld_recent=None):
        """Batched write-back of the reference's mutation (penalty, then / T)
        into device rows `logits` [B, ld]; stream-ordered, after
        sample_batch on the same rows."""
        B = int(logits.shape[0])
        V = int(logits.shape[1]) if V is None else V
        ld = (int(logits.stride(0)) if B > 1 else V) if ld is None else ld
        if recent is not None:
            W = int(recent.shape[1]) if W is None else W
            if ld_recent is None:
                ld_recent = int(recent.stride(0)) if recent.shape[0] > 1 else W
        else:
            W, ld_recent = 0, 0
        _check(self._lib.gs_logits_writeback(self._h, _ptr(logits), B, V, ld, _ptr(params), _ptr(recent),
                                             ld_recent, _ptr(recent_len), W, _stream_handle(stream)),
               "gs_logits_writeback")

    def sample_detail(self, logits, tokens, cap, params=None, recent=None, recent_len=None, u=None,
                      status=None, stream=None):
        """gs_sample_detail: the tokens of sample_batch plus, per row, the
        kept candidates (ids, post-softmax p; the first `cap`), n_kept, the
        nucleus cut, (S, s2) and the tie flag.  Returns a dict of device
        tensors; rows with T > 0 are sorted (slow)."""
        import torch
        B, V = int(logits.shape[0]), int(logits.shape[1])
        ld = int(logits.stride(0)) if B > 1 else V
        dev = logits.device
        out = {"ids": torch.zeros((B, cap), dtype=torch.int32, device=dev),
               "p": torch.zeros((B, cap), dtype=torch.float32, device=dev),
               "n_kept": torch.zeros(B, dtype=torch.int32, device=dev),
               "cut": torch.zeros(B, dtype=torch.int32, device=dev),
               "sums": torch.zeros((B, 2), dtype=torch.float32, device=dev),
               "ties": torch.zeros(B, dtype=torch.int32, device=dev)}
        det = GsDetail(_ptr(out["ids"]), _ptr(out["p"]), cap, _ptr(out["n_kept"]), _ptr(out["cut"]),
                       _ptr(out["sums"]), _ptr(out["ties"]))
        if recent is not None:
            W = int(recent.shape[1])
            ld_recent = int(recent.stride(0)) if recent.shape[0] > 1 else W
        else:
            W, ld_recent = 0, 0
        _check(self._lib.gs_sample_detail(self._h, _ptr(logits), B, V, ld, _ptr(params), _ptr(recent), ld_recent,
                                          _ptr(recent_len), W, _ptr(u), _ptr(tokens), _ptr(status),
                                          ctypes.byref(det), _stream_handle(stream)), "gs_sample_detail")
        return out

    def sample_batch(self, logits, tokens, params=None, recent=None, recent_len=None,
                     u=None, status=None, stream=None, V=None, ld=None, W=None, ld_recent=None,
                     noalloc=False):
        """Batched sampling over B device rows (torch tensors on cuda).
        logits [B, ld] f32; tokens [B] int32/uint32; params [B, 4]-shaped
        gs_params buffer (or None); recent [B, ld_recent] uint32 ids (or None);
        u [B] f32 draws (or None = this sampler's LCG stream).  Asynchronous.
        noalloc=True calls gs_sample_batch_noalloc (static scratch, no
        device allocation)."""
        B = int(logits.shape[0])
        V = int(logits.shape[1]) if V is None else V
        # a size-1 leading dimension may carry any stride (numpy gives 0)
        ld = (int(logits.stride(0)) if B > 1 else V) if ld is None else ld
        if recent is not None:
            W = int(recent.shape[1]) if W is None else W
            if ld_recent is None:
                ld_recent = int(recent.stride(0)) if recent.shape[0] > 1 else W
        else:
            W, ld_recent = 0, 0
        fn = self._lib.gs_sample_batch_noalloc if noalloc else self._lib.gs_sample_batch
        _check(fn(
            self._h, _ptr(logits), B, V, ld, _ptr(params), _ptr(recent), ld_recent,
            _ptr(recent_len), W, _ptr(u), _ptr(tokens), _ptr(status),
            _stream_handle(stream)), "gs_sample_batch_noalloc" if noalloc else "gs_sample_batch")


def window_push(window, tokens, pos, W=None, stream=None):
    lib = load_library()
    B = int(window.shape[0])
    W = int(window.shape[1]) if W is None else W
    ld = int(window.stride(0)) if B > 1 else int(window.shape[1])
    _check(lib.gs_window_push(_ptr(window), B, ld, W, pos, _ptr(tokens),
                              _stream_handle(stream)), "gs_window_push")


def synth_logits(out, seed, counter0, sigma, V=None, stream=None):
    lib = load_library()
    B = int(out.shape[0])
    V = int(out.shape[1]) if V is None else V
    ld = int(out.stride(0)) if B > 1 else int(out.shape[1])
    _check(lib.gs_synth_logits(_ptr(out), B, V, ld, seed, counter0, sigma,
                               _stream_handle(stream)), "gs_synth_logits")


def params_array(rows):
    """Pack [(T, top_k, top_p, rep), ...] as a numpy structured array whose
    bytes are B gs_params (16 bytes each)."""
    import numpy as np
    dt = np.dtype([("temperature", "<f4"), ("top_k", "<u4"), ("top_p", "<f4"), ("rep_penalty", "<f4")])
    return np.array([tuple(r) for r in rows], dtype=dt)


# ---- the reference's free-function API over a process-global sampler -----
_global = None
_global_seed = 12345  # src/sampler.rs:3


def _get_global():
    global _global
    if _global is None:
        _global = Sampler(0.7, 40, 0.9, 1.1, seed=_global_seed)
    return _global


def set_seed(s):
    """src/sampler.rs:5"""
    global _global_seed
    _global_seed = s
    if _global is not None:
        _global.set_seed(s)


def sample(logits, temperature, top_k, top_p, rep_penalty, recent):
    """src/sampler.rs:35-36 -- returns the token id.  Raises SamplerError
    where the reference panics."""
    g = _get_global()
    g.set_params(temperature, top_k, top_p, rep_penalty)
    return g.sample(logits, recent)


def sample_mut(logits, temperature, top_k, top_p, rep_penalty, recent):
    """sample() that also leaves `logits` mutated in place as the reference
    does (src/sampler.rs:37,41): penalized, then divided by T when T > 0."""
    g = _get_global()
    g.set_params(temperature, top_k, top_p, rep_penalty)
    return g.sample_mut(logits, recent)


# ---- quantized output projection (include/gs_gemv.h) --------------------------
QTYPE_Q4_0 = 2     # GgmlType::Q4_0 (src/gguf/types.rs:42)
QTYPE_Q4_1 = 3     # GgmlType::Q4_1
QTYPE_Q8_0 = 8     # GgmlType::Q8_0 (src/gguf/types.rs:43)
QTYPE_Q3_K = 11    # GgmlType::Q3K  (src/gguf/types.rs:44)
QTYPE_Q4_K = 12    # GgmlType::Q4K
QTYPE_Q5_K = 13    # GgmlType::Q5K
QTYPE_Q6_K = 14    # GgmlType::Q6K


class QMatrix:
    """A quantized matrix on the device: Gpu::upload (src/gpu/mod.rs:222-238)
    of a Q4_0 / Q4_1 / Q8_0 / Q3_K / Q4_K / Q5_K / Q6_K GGUF tensor.  `blocks` are the tensor's raw bytes (a
    numpy uint8 array or bytes), rows x cols weights, cols = dims[0].
    gemv(x, out) is Gpu::cmd_gemv (src/gpu/mod.rs:438-443): out = W x for
    device f32 vectors (torch tensors or device addresses), B = len(x) / cols
    vectors per call."""

    def __init__(self, qtype, blocks, rows, cols):
        import numpy as np
        self._lib = load_library()
        b = np.ascontiguousarray(np.frombuffer(blocks, dtype=np.uint8) if isinstance(blocks, (bytes, bytearray))
                                 else blocks, dtype=np.uint8)
        h = ctypes.c_void_p()
        _check(self._lib.gs_qmatrix_upload(qtype, b.ctypes.data, rows, cols, ctypes.byref(h)),
               "gs_qmatrix_upload")
        self._h = h
        self.qtype, self.rows, self.cols = qtype, rows, cols

    def gemv(self, x, out, B=1, stream=None):
        st = None
        if stream is not None:
            st = stream.cuda_stream if hasattr(stream, "cuda_stream") else stream
        _check(self._lib.gs_gemv(self._h, _ptr(x), B, _ptr(out), st), "gs_gemv")

    def close(self):
        if self._h:
            self._lib.gs_qmatrix_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- device-resident decode loop (include/gs_decode.h) ------------------------
DONE_RUNNING, DONE_STOP, DONE_MAX, DONE_ERROR = 0, 1, 2, 3


def decode_row_dtype():
    """numpy dtype of gs_decode_row (24 bytes)."""
    import numpy as np
    return np.dtype([("rng", "<u8"), ("n_gen", "<u4"), ("wpos", "<u4"), ("done", "<u4"), ("last", "<u4")])


class Decoder:
    """Device buffers of B decoding rows and the step of generate_collect
    (src/main.rs:279-311) over them: sample, stop check, max-length check,
    window push, generated push.  Buffers are torch tensors on cuda; every
    method is stream-ordered and, apart from init() and the read-outs,
    asynchronous."""

    def __init__(self, B, W=64, max_new=256, stop=(), device="cuda"):
        import torch
        self._lib = load_library()
        self.B, self.W, self.max_new = B, W, max_new
        dev = torch.device(device)
        u32 = torch.int32
        self.rows = torch.zeros(B * 24, dtype=torch.uint8, device=dev)
        self.window = torch.zeros((B, max(W, 1)), dtype=u32, device=dev)
        self.window_len = torch.zeros(B, dtype=u32, device=dev)
        stop = [int(s) for s in stop]
        self.stop = torch.tensor(stop if stop else [0], dtype=torch.int64).to(u32).to(dev)
        self.generated = torch.zeros((B, max(max_new, 1)), dtype=u32, device=dev)
        self.next = torch.zeros(B, dtype=u32, device=dev)
        self.u = torch.zeros(B, dtype=torch.float32, device=dev)
        self.tokens = torch.zeros(B, dtype=u32, device=dev)
        self.status = torch.zeros(B, dtype=torch.int32, device=dev)
        self.n_active = torch.zeros(1, dtype=u32, device=dev)
        self.ctx = DecodeCtx(B, self.rows.data_ptr(), self.window.data_ptr() if W else None,
                             self.window.stride(0), W, self.window_len.data_ptr() if W else None,
                             self.stop.data_ptr() if stop else None, len(stop), max_new,
                             self.generated.data_ptr(), self.generated.stride(0), self.next.data_ptr(),
                             self.u.data_ptr(), self.tokens.data_ptr(), self.status.data_ptr(),
                             self.n_active.data_ptr())

    def init(self, sampler, seeds, init_recent=None, params=None, stream=None):
        """Reset every row: LCG state = seeds[b] (set_seed, src/sampler.rs:5)
        and the window holding init_recent[b] (the reference's `recent` at
        the start of a turn, oldest first; at most W ids); then the first
        step's draws with the rows' temperatures (params: device gs_params
        per row, or None = the sampler's)."""
        import numpy as np
        import torch
        sd = np.ascontiguousarray(np.asarray(seeds, dtype=np.uint64).reshape(self.B))
        ln = np.zeros(self.B, np.uint32)
        if init_recent is not None:
            for b, r in enumerate(init_recent):
                r = np.asarray(r, dtype=np.uint32)
                if r.size > self.W:
                    raise ValueError("init_recent row %d longer than W" % b)
                ln[b] = r.size
                if r.size:
                    self.window[b, :r.size] = torch.from_numpy(r.view(np.int32)).to(self.window.device)
        _check(self._lib.gs_decode_init(sampler._h, _ptr(params), ctypes.byref(self.ctx), sd.ctypes.data,
                                        ln.ctypes.data, _stream_handle(stream)), "gs_decode_init")

    def step(self, sampler, logits=None, lm_head=None, x=None, params=None, stream=None):
        """One step.  Either lm_head (a QMatrix) and x [B, cols] f32 with
        `logits` a [B, rows] f32 output buffer, or logits [B, ld] holding
        this step's logits."""
        V = lm_head.rows if lm_head is not None else int(logits.shape[1])
        ld = V if lm_head is not None else (int(logits.stride(0)) if self.B > 1 else V)
        _check(self._lib.gs_decode_step(sampler._h, lm_head._h if lm_head is not None else None,
                                        _ptr(x), _ptr(logits), V, ld, _ptr(params), ctypes.byref(self.ctx),
                                        _stream_handle(stream)), "gs_decode_step")

    def commit(self, sampler, params=None, stream=None):
        """gs_decode_commit: commit self.tokens (sampled by the caller) and
        draw the next step's u."""
        _check(self._lib.gs_decode_commit(sampler._h, _ptr(params), ctypes.byref(self.ctx),
                                          _stream_handle(stream)), "gs_decode_commit")

    def row_state(self):
        """The B gs_decode_row records, copied to the host (synchronises)."""
        import numpy as np
        return self.rows.cpu().numpy().view(decode_row_dtype()).copy()

    def generated_ids(self):
        """Per row, the generated ids (list of numpy uint32 arrays)."""
        st = self.row_state()
        g = self.generated.cpu().numpy().view("<u4")
        return [g[b, :min(int(st["n_gen"][b]), g.shape[1])].copy() for b in range(self.B)]


# ---- token text and stop set (include/gs_tokens.h) -----------------------------
TOK_LLAMA, TOK_GPT2 = 0, 1
TMPL_CHATML, TMPL_LLAMA3, TMPL_LLAMA2, TMPL_GEMMA, TMPL_PHI3, TMPL_SIMPLE = range(6)


class Vocab:
    """The tokenizer's vocabulary for the text step after the sampler:
    decode(id) is Tokenizer::decode (src/tokenizer/bpe.rs:180-197),
    detect / stop_tokens are ChatTemplate's (src/tokenizer/chat.rs:9-72).
    `tokens` are str or bytes; `types` the GGUF token types; `model` is
    TOK_LLAMA or TOK_GPT2.  Host-only."""

    def __init__(self, tokens, types=(), model=TOK_LLAMA):
        import numpy as np
        self._lib = load_library()
        raw = [t.encode("utf-8") if isinstance(t, str) else bytes(t) for t in tokens]
        off = np.zeros(len(raw) + 1, np.uint64)
        off[1:] = np.cumsum([len(r) for r in raw], dtype=np.uint64)
        data = b"".join(raw)
        ty = np.ascontiguousarray(np.asarray(types, dtype=np.uint32))
        self._data = ctypes.create_string_buffer(data, max(len(data), 1))
        h = ctypes.c_void_p()
        _check(self._lib.gs_vocab_create(self._data, off.ctypes.data, len(raw),
                                         ty.ctypes.data if ty.size else None, ty.size, model,
                                         ctypes.byref(h)), "gs_vocab_create")
        self._h = h

    def find(self, s):
        b = s.encode("utf-8") if isinstance(s, str) else bytes(s)
        out = ctypes.c_uint32()
        _check(self._lib.gs_vocab_find(self._h, b, len(b), ctypes.byref(out)), "gs_vocab_find")
        return None if out.value == 0xFFFFFFFF else int(out.value)

    def decode_bytes(self, ids):
        """The UTF-8 bytes of decode(id) concatenated over ids (an int or a sequence)."""
        import numpy as np
        a = np.ascontiguousarray(np.atleast_1d(np.asarray(ids, dtype=np.uint32)))
        n = ctypes.c_size_t()
        _check(self._lib.gs_tokens_decode(self._h, a.ctypes.data, a.size, None, 0, ctypes.byref(n)),
               "gs_tokens_decode")
        buf = ctypes.create_string_buffer(max(n.value, 1))
        _check(self._lib.gs_tokens_decode(self._h, a.ctypes.data, a.size, buf, n.value, ctypes.byref(n)),
               "gs_tokens_decode")
        return buf.raw[:n.value]

    def decode(self, ids):
        return self.decode_bytes(ids).decode("utf-8")

    def detect(self, tmpl=None):
        out = ctypes.c_uint32()
        _check(self._lib.gs_chat_template_detect(self._h, None if tmpl is None else tmpl.encode("utf-8"),
                                                 ctypes.byref(out)), "gs_chat_template_detect")
        return int(out.value)

    def stop_tokens(self, kind, eos_ids):
        import numpy as np
        e = np.ascontiguousarray(np.asarray(eos_ids, dtype=np.uint32))
        n = ctypes.c_size_t()
        out = np.zeros(len(eos_ids) + 8, np.uint32)
        _check(self._lib.gs_stop_tokens(self._h, kind, e.ctypes.data if e.size else None, e.size,
                                        out.ctypes.data, out.size, ctypes.byref(n)), "gs_stop_tokens")
        return [int(x) for x in out[:n.value]]

    def close(self):
        if self._h:
            self._lib.gs_vocab_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
