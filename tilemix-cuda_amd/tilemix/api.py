"""ctypes binding of include/tilemix_capi.h (see the package docstring)."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Optional

SUCCESS = 0
ERROR_INVALID_VALUE = 1
ERROR_INVALID_CONFIGURATION = 9
ERROR_NOT_SUPPORTED = 801

_PACKAGE_DIR = Path(__file__).resolve().parent.parent
_LIB_NAME = "libtilemix_hip.so"
_lib: Optional[ctypes.CDLL] = None


class TileMixError(RuntimeError):
    def __init__(self, code: int, what: str = ""):
        super().__init__(f"TileMix call failed with hipError_t {code}{': ' + what if what else ''}")
        self.code = code


def library_path() -> Path:
    """The in-tree build (tilemix-cuda_amd/libtilemix_hip.so)."""
    return _PACKAGE_DIR / _LIB_NAME


# Element types of O (include/tilemix_capi.h TILEMIX_DTYPE_*).
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2


class _BatchedArgs(ctypes.Structure):
    _fields_ = [
        ("Q", ctypes.c_void_p), ("K", ctypes.c_void_p), ("V", ctypes.c_void_p), ("O", ctypes.c_void_p),
        ("heads", ctypes.c_int), ("M", ctypes.c_int), ("N", ctypes.c_int), ("d", ctypes.c_int),
        ("q_head_stride", ctypes.c_int64), ("k_head_stride", ctypes.c_int64),
        ("v_head_stride", ctypes.c_int64), ("o_head_stride", ctypes.c_int64),
        ("score_scale", ctypes.c_float), ("causal", ctypes.c_int), ("precise", ctypes.c_int),
        ("quantize", ctypes.c_int),
        ("route_words", ctypes.c_void_p), ("skip_words", ctypes.c_void_p),
        ("key_tiles_per_group", ctypes.c_int), ("decoded_bits", ctypes.c_void_p),
        ("Q8", ctypes.c_void_p), ("K8", ctypes.c_void_p), ("q_scales", ctypes.c_void_p),
        ("k_scales", ctypes.c_void_p), ("score_dots", ctypes.c_void_p),
        ("o_dtype", ctypes.c_int), ("q_row_stride", ctypes.c_int64), ("k_row_stride", ctypes.c_int64),
        ("v_row_stride", ctypes.c_int64), ("o_row_stride", ctypes.c_int64),
    ]


def library() -> ctypes.CDLL:
    """Load libtilemix_hip.so (built by tilemix-cuda_amd/build.py); raises if absent."""
    global _lib
    if _lib is None:
        # PyTorch bundles its own HIP runtime (same SONAME, libamdhip64.so.7).
        # Loading torch first makes the dynamic linker bind this library to
        # that one runtime, so torch tensors and streams are valid here.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        path = library_path()
        if not path.exists():
            raise ImportError(f"{path} is missing: build it with `python tilemix-cuda_amd/build.py` "
                              "(there is no fallback implementation)")
        so = ctypes.CDLL(str(path))
        vp, i32, i64, sz, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float
        so.tilemix_quantize_qk.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, i32, vp]
        so.tilemix_quantize_qk.restype = i32
        so.tilemix_attention.argtypes = [vp, vp, vp, vp, i32, i32, i32, f32, vp, vp, sz, i32, vp,
                                         vp, vp, vp, vp, vp]
        so.tilemix_attention.restype = i32
        so.tilemix_attention_batched.argtypes = [ctypes.POINTER(_BatchedArgs), vp]
        so.tilemix_attention_batched.restype = i32
        so.tilemix_quantize_qk_batched.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i64, i64, vp]
        so.tilemix_quantize_qk_batched.restype = i32
        so.tilemix_quantize_qk_strided.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i64, i64, i64, i64,
                                                   vp]
        so.tilemix_quantize_qk_strided.restype = i32
        so.tilemix_routing_words_per_row_c.argtypes = [i32, i32]
        so.tilemix_routing_words_per_row_c.restype = sz
        so.tilemix_routing_word_count_c.argtypes = [i32, i32, i32]
        so.tilemix_routing_word_count_c.restype = sz
        so.tilemix_shared_bytes_c.argtypes = [i32, i32]
        so.tilemix_shared_bytes_c.restype = sz
        so.tilemix_version.argtypes = []
        so.tilemix_version.restype = ctypes.c_char_p
        u64 = ctypes.c_uint64
        so.tilemix_routes_from_tiles.argtypes = [vp, i32, i32, i32, i32, i32, i32, vp, vp, vp]
        so.tilemix_routes_from_tiles.restype = i32
        so.tilemix_tiles_bernoulli.argtypes = [vp, i32, i32, i32, i32, i32, f32, u64, vp]
        so.tilemix_tiles_bernoulli.restype = i32
        so.tilemix_tiles_causal_band.argtypes = [vp, i32, i32, i32, i32, i32, f32, u64, vp]
        so.tilemix_tiles_causal_band.restype = i32
        so.tilemix_tiles_three_way.argtypes = [vp, i32, i32, i32, i32, i32, f32, f32, u64, vp]
        so.tilemix_tiles_three_way.restype = i32
        so.tilemix_importance_workspace_bytes.argtypes = [i32, i32, i32, i32, i32]
        so.tilemix_importance_workspace_bytes.restype = sz
        so.tilemix_tiles_importance.argtypes = [vp, vp, i32, i32, i32, i32, i64, i64, i32, i32, f32, vp, sz,
                                                vp, vp]
        so.tilemix_tiles_importance.restype = i32
        so.tilemix_importance_noalloc_max_bytes.argtypes = []
        so.tilemix_importance_noalloc_max_bytes.restype = sz
        so.tilemix_tiles_importance_noalloc.argtypes = [vp, vp, i32, i32, i32, i32, i64, i64, i32, i32, f32, vp, vp]
        so.tilemix_tiles_importance_noalloc.restype = i32
        _lib = so
    return _lib


def _ptr(x: Any) -> Optional[int]:
    """Device address of a torch tensor, an int address, or None (NULL)."""
    if x is None:
        return None
    if isinstance(x, int):
        return x or None
    return x.data_ptr() or None


def _stream(stream: Any) -> Optional[int]:
    """hipStream_t of `stream`: a torch stream, an int handle (0 = the null
    stream), or None = torch's current stream on the current device (as torch
    ops would use), so that a call inside `with torch.cuda.stream(s):` is
    ordered after the kernels that produced its inputs. Before torch has
    initialised the GPU no torch stream can be current: None is then the null
    stream."""
    if stream is None:
        import sys

        torch = sys.modules.get("torch")
        if torch is None or not torch.cuda.is_initialized():
            return None
        return torch.cuda.current_stream().cuda_stream or None
    if isinstance(stream, int):
        return stream or None
    return stream.cuda_stream or None


def check(code: int, what: str = "") -> None:
    if code != SUCCESS:
        raise TileMixError(code, what)


def version() -> str:
    return library().tilemix_version().decode()


def routing_words_per_row(N: int, key_tiles_per_group: int) -> int:
    return int(library().tilemix_routing_words_per_row_c(N, key_tiles_per_group))


def routing_word_count(M: int, N: int, key_tiles_per_group: int) -> int:
    return int(library().tilemix_routing_word_count_c(M, N, key_tiles_per_group))


def shared_bytes(d: int, quantized: bool) -> int:
    return int(library().tilemix_shared_bytes_c(d, int(bool(quantized))))


@dataclass
class TileMixRouting:
    """include/attention_fused.h:47-52 (words: uint64 device tensor, bit 1 = INT8)."""
    words: Any = None
    word_count: int = 0
    key_tiles_per_group: int = 1
    decoded_bits: Any = None


@dataclass
class TileMixQuantized:
    """include/attention_fused.h:54-60."""
    q: Any = None
    k: Any = None
    q_scales: Any = None
    k_scales: Any = None
    score_dots: Any = None


def quantize_tilemix_qk(Q, K, Q8, K8, q_scales, k_scales, M: int, N: int, d: int, stream=None) -> int:
    """Reference quantize_tilemix_qk (attention_fused.h:62-65); returns the hipError_t code."""
    return library().tilemix_quantize_qk(_ptr(Q), _ptr(K), _ptr(Q8), _ptr(K8), _ptr(q_scales),
                                         _ptr(k_scales), M, N, d, _stream(stream))


def launch_fused_fp16_attention(Q, K, V, O, M: int, N: int, d: int, score_scale: float, stream=None,
                                routing: Optional[TileMixRouting] = None,
                                quantized: Optional[TileMixQuantized] = None) -> int:
    """Reference launch_fused_fp16_attention (attention_fused.h:68-72); returns the hipError_t code."""
    r = routing or TileMixRouting()
    qz = quantized or TileMixQuantized()
    return library().tilemix_attention(
        _ptr(Q), _ptr(K), _ptr(V), _ptr(O), M, N, d, ctypes.c_float(score_scale), _stream(stream),
        _ptr(r.words), r.word_count, r.key_tiles_per_group, _ptr(r.decoded_bits),
        _ptr(qz.q), _ptr(qz.k), _ptr(qz.q_scales), _ptr(qz.k_scales), _ptr(qz.score_dots))


@dataclass
class BatchedArgs:
    """Multi-head problem of tilemix_attention_batched (TileMixBatchedArgs)."""
    Q: Any
    K: Any
    V: Any
    O: Any
    heads: int
    M: int
    N: int
    d: int
    score_scale: float
    q_head_stride: int = 0
    k_head_stride: int = 0
    v_head_stride: int = 0
    o_head_stride: int = 0
    causal: bool = False
    precise: bool = False
    quantize: int = 1  # 0: Q8/K8 given, 1: quantize Q and K, 2: K8 given, quantize Q
    route_words: Any = None
    skip_words: Any = None
    key_tiles_per_group: int = 1
    decoded_bits: Any = None
    Q8: Any = None
    K8: Any = None
    q_scales: Any = None
    k_scales: Any = None
    score_dots: Any = None
    o_dtype: int = 0  # DTYPE_F32, DTYPE_F16 or DTYPE_BF16
    q_row_stride: int = 0  # elements between rows of a head, 0 = d
    k_row_stride: int = 0
    v_row_stride: int = 0
    o_row_stride: int = 0

    def to_c(self) -> _BatchedArgs:
        qn, kn = self.M * self.d, self.N * self.d
        return _BatchedArgs(
            _ptr(self.Q), _ptr(self.K), _ptr(self.V), _ptr(self.O), self.heads, self.M, self.N, self.d,
            self.q_head_stride or qn, self.k_head_stride or kn, self.v_head_stride or kn,
            self.o_head_stride or qn, ctypes.c_float(self.score_scale), int(self.causal),
            int(self.precise), int(self.quantize), _ptr(self.route_words), _ptr(self.skip_words),
            self.key_tiles_per_group, _ptr(self.decoded_bits), _ptr(self.Q8), _ptr(self.K8),
            _ptr(self.q_scales), _ptr(self.k_scales), _ptr(self.score_dots), int(self.o_dtype),
            self.q_row_stride, self.k_row_stride, self.v_row_stride, self.o_row_stride)


def attention_batched(args: BatchedArgs, stream=None) -> int:
    """tilemix_attention_batched; returns the hipError_t code."""
    c_args = args.to_c()
    return library().tilemix_attention_batched(ctypes.byref(c_args), _stream(stream))


def quantize_tilemix_qk_strided(Q, K, Q8, K8, q_scales, k_scales, heads: int, M: int, N: int, d: int,
                                q_head_stride: int = 0, k_head_stride: int = 0, q_row_stride: int = 0,
                                k_row_stride: int = 0, stream=None) -> int:
    return library().tilemix_quantize_qk_strided(
        _ptr(Q), _ptr(K), _ptr(Q8), _ptr(K8), _ptr(q_scales), _ptr(k_scales), heads, M, N, d,
        q_head_stride or M * d, k_head_stride or N * d, q_row_stride, k_row_stride, _stream(stream))


def quantize_tilemix_qk_batched(Q, K, Q8, K8, q_scales, k_scales, heads: int, M: int, N: int, d: int,
                                q_head_stride: int = 0, k_head_stride: int = 0, stream=None) -> int:
    return library().tilemix_quantize_qk_batched(
        _ptr(Q), _ptr(K), _ptr(Q8), _ptr(K8), _ptr(q_scales), _ptr(k_scales), heads, M, N, d,
        q_head_stride or M * d, k_head_stride or N * d, _stream(stream))


# ------------------------------------------------------- device mask producer
# Extensions with no reference counterpart (the reference builds masks on
# the host, src/tests/tilemix_test.cu:432-448): tile codes [heads, tiles_q,
# tiles_k] uint8 (0 FP16, 1 INT8, 2 skip) built on the GPU, then packed into
# the TileMixRouting word format (include/attention_fused.h:34-52).


def routes_from_tiles(tile_codes, heads: int, M: int, N: int, tile_rows: int, tile_keys: int,
                      key_tiles_per_group: int, route_words, skip_words, stream=None) -> int:
    return library().tilemix_routes_from_tiles(_ptr(tile_codes), heads, M, N, tile_rows, tile_keys,
                                               key_tiles_per_group, _ptr(route_words), _ptr(skip_words),
                                               _stream(stream))


def tiles_bernoulli(tile_codes, heads: int, M: int, N: int, tile_rows: int, tile_keys: int, p_int8: float,
                    seed: int, stream=None) -> int:
    return library().tilemix_tiles_bernoulli(_ptr(tile_codes), heads, M, N, tile_rows, tile_keys, p_int8,
                                             seed, _stream(stream))


def tiles_causal_band(tile_codes, heads: int, S: int, tile_rows: int, tile_keys: int, fp16_band: int,
                      p_int8: float, seed: int, stream=None) -> int:
    return library().tilemix_tiles_causal_band(_ptr(tile_codes), heads, S, tile_rows, tile_keys, fp16_band,
                                               p_int8, seed, _stream(stream))


def tiles_three_way(tile_codes, heads: int, M: int, N: int, tile_rows: int, tile_keys: int, p_skip: float,
                    p_int8: float, seed: int, stream=None) -> int:
    return library().tilemix_tiles_three_way(_ptr(tile_codes), heads, M, N, tile_rows, tile_keys, p_skip,
                                             p_int8, seed, _stream(stream))


def importance_workspace_bytes(heads: int, M: int, N: int, tile_rows: int, tile_keys: int) -> int:
    return library().tilemix_importance_workspace_bytes(heads, M, N, tile_rows, tile_keys)


def tiles_importance(Q, K, heads: int, M: int, N: int, d: int, tile_rows: int, tile_keys: int,
                     fp16_fraction: float, workspace, workspace_bytes: int, tile_codes,
                     q_head_stride: int = 0, k_head_stride: int = 0, stream=None) -> int:
    return library().tilemix_tiles_importance(_ptr(Q), _ptr(K), heads, M, N, d, q_head_stride or M * d,
                                              k_head_stride or N * d, tile_rows, tile_keys, fp16_fraction,
                                              _ptr(workspace), workspace_bytes, _ptr(tile_codes),
                                              _stream(stream))


def importance_noalloc_max_bytes() -> int:
    """Size of the library's fixed scratch used by tiles_importance_noalloc."""
    return int(library().tilemix_importance_noalloc_max_bytes())


def tiles_importance_noalloc(Q, K, heads: int, M: int, N: int, d: int, tile_rows: int, tile_keys: int,
                             fp16_fraction: float, tile_codes, q_head_stride: int = 0, k_head_stride: int = 0,
                             stream=None) -> int:
    """tiles_importance without a workspace (the library's fixed scratch; the
    call allocates no device memory). Calls that overlap on one GPU race."""
    return library().tilemix_tiles_importance_noalloc(_ptr(Q), _ptr(K), heads, M, N, d, q_head_stride or M * d,
                                                      k_head_stride or N * d, tile_rows, tile_keys,
                                                      fp16_fraction, _ptr(tile_codes), _stream(stream))
