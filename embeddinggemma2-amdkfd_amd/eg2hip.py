"""Python binding of libeg2hip.so (the gfx950 executor and its operators).

Mirrors the reference's executor interface (src/gemma2_kfd.h:7-10):
`Encoder(gguf_path)` wraps ei_gemma2_kfd_create / _free and
`Encoder.batch(ids, offsets)` wraps ei_gemma2_kfd_batch, raising on the
same conditions the C ABI reports with `false` + message. `ops` exposes the
operator-level entry points of include/eg2_hip.h for device buffers (torch
tensors are used only as device allocations and for their streams).

The library must be built (`make -C embeddinggemma2-amdkfd_amd`); there is
no fallback path: a missing library raises immediately.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libeg2hip.so")

N_EMBD, N_FF, HEAD_DIM, N_CTX, VOCAB = 768, 1152, 256, 2048, 262144
QKV_COLS = N_EMBD + 2 * HEAD_DIM

_vp, _f, _i32 = C.c_void_p, C.POINTER(C.c_float), C.POINTER(C.c_int32)
_u = C.c_uint


class EiStr(C.Structure):
    _fields_ = [("str", C.c_void_p), ("len", C.c_uint64)]


class _KvValue(C.Union):
    _fields_ = [("u64", C.c_uint64), ("i64", C.c_int64), ("f64", C.c_double), ("b", C.c_bool), ("s", EiStr)]


class EiKv(C.Structure):
    _fields_ = [("key", EiStr), ("type", C.c_uint32), ("v", _KvValue), ("arr_type", C.c_uint32),
                ("arr_n", C.c_uint64), ("arr_data", C.c_void_p)]


class EiTensor(C.Structure):
    _fields_ = [("name", EiStr), ("n_dims", C.c_uint32), ("ne", C.c_uint64 * 4), ("type", C.c_uint32),
                ("offset", C.c_uint64), ("data", C.c_void_p), ("n_bytes", C.c_uint64)]


class EiGguf(C.Structure):
    _fields_ = [("map", C.c_void_p), ("map_len", C.c_size_t), ("version", C.c_uint32), ("n_kv", C.c_uint64),
                ("n_tensors", C.c_uint64), ("alignment", C.c_uint64), ("data_off", C.c_uint64),
                ("kv", C.POINTER(EiKv)), ("tensors", C.POINTER(EiTensor))]


class BatchConfig(C.Structure):
    """eg2_batch_config (include/eg2_stream.h)."""
    _fields_ = [("max_batch_tokens", C.c_size_t), ("max_batch_sequence_tokens", C.c_size_t),
                ("max_batch_requests", C.c_size_t), ("lookahead", C.c_uint), ("sort_longest_first", C.c_uint)]


class SynthConfig(C.Structure):
    _fields_ = [("seed", C.c_uint64), ("n_layer", C.c_uint), ("dense_head", C.c_uint), ("weight_std", C.c_float),
                ("embed_std", C.c_float), ("norm_std", C.c_float), ("rope_base_full", C.c_float),
                ("rope_base_swa", C.c_float), ("sliding_window", C.c_uint), ("sliding_window_pattern", C.c_uint),
                ("threads", C.c_uint)]


# The operator records of include/abi.h (kernels/abi.h:3-11) and EgSaxpy.
class EgGather(C.Structure):
    _fields_ = [("out", _vp), ("weight", _vp), ("ids", _vp), ("n", _u)]


class EgMM(C.Structure):
    _fields_ = [("out", _vp), ("x", _vp), ("weight", _vp), ("n", _u), ("k", _u), ("m", _u), ("type", _u)]


class EgNorm(C.Structure):
    _fields_ = [("out", _vp), ("x", _vp), ("weight", _vp), ("rows", _u), ("d", _u), ("scale", C.c_float)]


class EgRope(C.Structure):
    _fields_ = [("x", _vp), ("table", _vp), ("n", _u), ("heads", _u), ("d", _u)]


class EgAttention(C.Structure):
    _fields_ = [("out", _vp), ("q", _vp), ("k", _vp), ("v", _vp), ("bounds", _vp), ("n", _u), ("window", _u)]


class EgElement(C.Structure):
    _fields_ = [("out", _vp), ("x", _vp), ("other", _vp), ("n", _u), ("mode", _u), ("layer", _u),
                ("scale", C.c_float)]


class EgPool(C.Structure):
    _fields_ = [("out", _vp), ("x", _vp), ("offsets", _vp), ("batch", _u)]


class EgNormResidual(C.Structure):
    _fields_ = [("out", _vp), ("x", _vp), ("weight", _vp), ("rows", _u), ("d", _u), ("scale", C.c_float)]


class EgNormRope(C.Structure):
    _fields_ = [("x", _vp), ("weight", _vp), ("table", _vp), ("rows", _u), ("d", _u), ("heads", _u)]


class EgSaxpy(C.Structure):
    _fields_ = [("y", _vp), ("x", _vp), ("a", C.c_float), ("n", _u)]


# Every symbol declared in include/eg2_hip.h, eg2_ops.h, eg2_stream.h and gemma2_kfd.h.
SIGNATURES = {
    "eg2_op_launch": (C.c_int, [C.c_char_p, _vp, C.c_size_t, _u, _u, _u, _vp]),
    "eg2_op_count": (C.c_uint, []),
    "eg2_op_name": (C.c_char_p, [_u]),
    "eg2_hip_embed_norm_quant": (C.c_int, [_vp, _vp, _u, C.c_float, _vp, C.c_float, _vp, _vp, _vp, _vp]),
    "eg2_hip_residual_norm_quant": (C.c_int, [_vp, _vp, _vp, _vp, C.c_float, _vp, _vp, _u, _vp]),
    "eg2_hip_qk_norm_rope": (C.c_int, [_vp, _vp, _vp, _vp, _vp, C.c_float, _vp, _u, _vp]),
    "eg2_hip_attention": (C.c_int, [_vp, _vp, _vp, _u, _vp, _u, _u, _u, _vp, _vp, _vp, _vp]),
    "eg2_hip_attention_static": (C.c_int, [_vp, _vp, _u, _u, _u, _vp, _vp, _vp]),
    "eg2_hip_attention_scores": (C.c_int, [_vp, _vp, _vp, _u, _u, _u, _vp, _vp]),
    "eg2_hip_attention_softmax": (C.c_int, [_vp, _u, _u, _u, _vp, _vp]),
    "eg2_hip_attention_context": (C.c_int, [_vp, _vp, _vp, _u, _u, _u, _vp, _vp, _vp, _vp]),
    "eg2_attention_plan": (C.c_int, [C.POINTER(C.c_size_t), C.c_size_t, C.c_size_t, C.c_size_t, _vp, _vp,
                                     C.POINTER(C.c_size_t)]),
    "eg2_attention_capacity": (None, [C.c_size_t, C.c_size_t, C.POINTER(C.c_size_t)]),
    "eg2_hip_gelu_quant": (C.c_int, [_vp, _vp, _vp, _u, _vp]),
    "eg2_hip_libm_eval": (C.c_int, [_vp, _u, _vp, _vp, _vp]),
    "eg2_hip_tanh_approx_error": (C.c_int, [_vp, _vp]),
    "eg2_hip_quantize_rows": (C.c_int, [_vp, _u, _vp, _vp, _u, _vp]),
    "eg2_hip_rms_norm_rows": (C.c_int, [_vp, _vp, C.c_float, _u, _vp]),
    "eg2_hip_pool_l2": (C.c_int, [_vp, _vp, _vp, _u, _vp]),
    "eg2_hip_pool_mean": (C.c_int, [_vp, _vp, _vp, _u, _vp]),
    "eg2_hip_l2_prefix": (C.c_int, [_vp, _u, _u, _u, _vp]),
    "eg2_hip_gemm_q8": (C.c_int, [_vp, _vp, _u, _vp, _vp, _u, _vp, _u, _u, _u, _u, _vp]),
    "eg2_hip_gemm_q8_geglu": (C.c_int, [_vp, _vp, _u, _vp, _vp, _u, _vp, _vp, _u, _u, _u, _u, _vp]),
    "eg2_hip_gemm_q8_qkv_rope": (C.c_int, [_vp, _vp, _u, _vp, _vp, _u, _u, _u, _vp, _vp, _vp, _vp, C.c_float, _vp,
                                           _vp]),
    "eg2_hip_error_string": (C.c_char_p, [C.c_int]),
    "eg2_hip_device_check": (C.c_int, [C.c_char_p, C.c_size_t]),
    "eg2_q8_tile_bytes": (C.c_size_t, [C.c_size_t, _u]),
    "eg2_q8_pack_rows": (None, [_vp, C.c_size_t, _u, _vp]),
    "eg2_q8_unpack_rows": (None, [_vp, C.c_size_t, _u, _vp]),
    "eg2_q8_weight_tiles": (None, [_vp, C.c_size_t, _u, _vp, _vp]),
    "eg2_q8_geglu_weight_tiles": (C.c_int, [_vp, _vp, C.c_size_t, _u, _vp, _vp]),
    "eg2_rope_table": (None, [C.c_float, _u, _vp]),
    "eg2_gguf_open": (C.c_int, [C.c_char_p, C.POINTER(EiGguf), C.c_char_p, C.c_size_t]),
    "eg2_gguf_close": (None, [C.POINTER(EiGguf)]),
    "eg2_synth_write_gguf": (C.c_int, [C.c_char_p, C.POINTER(SynthConfig), C.c_char_p, C.c_size_t]),
    "eg2_batch_config_default": (None, [C.POINTER(BatchConfig)]),
    "eg2_pack_waves": (C.c_size_t, [C.POINTER(C.c_size_t), C.c_size_t, C.POINTER(BatchConfig), C.POINTER(C.c_size_t),
                                    C.POINTER(C.c_size_t)]),
    "eg2_normalize_prefix": (C.c_bool, [_f, C.c_uint]),
    "eg2_stream_embed": (C.c_bool, [C.c_void_p, _i32, C.POINTER(C.c_size_t), C.c_size_t, C.POINTER(C.c_uint),
                                    C.POINTER(BatchConfig), _f, C.POINTER(C.c_size_t), C.c_char_p, C.c_size_t]),
    "ei_gemma2_kfd_create": (C.c_void_p, [C.POINTER(EiGguf), C.c_char_p, C.c_size_t]),
    "ei_gemma2_kfd_free": (None, [C.c_void_p]),
    "eg2_kfd_stage": (C.c_bool, [C.c_void_p, _i32, C.POINTER(C.c_size_t), C.c_size_t, C.c_char_p, C.c_size_t]),
    "eg2_kfd_launch_staged": (C.c_bool, [C.c_void_p, C.c_uint, C.c_char_p, C.c_size_t]),
    "eg2_kfd_collect": (C.c_bool, [C.c_void_p, _f, C.c_char_p, C.c_size_t]),
    "eg2_kfd_lanes": (C.c_uint, [C.c_void_p]),
    "eg2_kfd_validate_gguf": (C.c_bool, [C.POINTER(EiGguf), C.c_char_p, C.c_size_t]),
    "eg2_kfd_inject_failure": (None, [C.c_void_p]),
    "eg2_f32_to_chars": (C.c_size_t, [C.c_char_p, C.c_float]),
    "eg2_tokenizer_create": (C.c_void_p, [C.c_void_p, C.c_char_p, C.c_size_t]),
    "eg2_tokenizer_free": (None, [C.c_void_p]),
    "eg2_tokenizer_text_to_id": (C.c_int32, [C.c_void_p, C.c_char_p, C.c_size_t]),
    "eg2_tokenize": (C.c_size_t, [C.c_void_p, C.c_char_p, C.c_size_t, C.c_bool, C.c_bool, _i32, C.c_size_t]),
    "eg2_tokenize_batch": (C.c_size_t, [C.c_void_p, C.c_char_p, C.POINTER(C.c_size_t), C.c_size_t, C.c_bool,
                                        C.c_bool, _i32, C.c_size_t, C.POINTER(C.c_size_t), C.c_uint]),
    "eg2_base64_f32": (C.c_size_t, [_f, C.c_size_t, C.c_char_p]),
    "eg2_embeddings_response_bound": (C.c_size_t, [C.c_size_t, C.c_uint, C.c_size_t]),
    "eg2_embeddings_response": (C.c_size_t, [_f, C.c_size_t, C.c_uint, C.c_int, C.c_int, C.c_char_p, C.c_size_t,
                                             C.c_size_t, C.c_char_p, C.c_size_t]),
    "eg2_kfd_acquire_lane": (C.c_int, [C.c_void_p]),
    "eg2_kfd_try_acquire_lane": (C.c_int, [C.c_void_p]),
    "eg2_kfd_release_lane": (None, [C.c_void_p, C.c_uint]),
    "eg2_kfd_stage_lane": (C.c_bool, [C.c_void_p, C.c_uint, _i32, C.POINTER(C.c_size_t), C.c_size_t, C.c_char_p,
                                      C.c_size_t]),
    "eg2_kfd_launch_lane": (C.c_bool, [C.c_void_p, C.c_uint, C.c_uint, C.c_char_p, C.c_size_t]),
    "eg2_kfd_collect_lane": (C.c_bool, [C.c_void_p, C.c_uint, _f, C.c_char_p, C.c_size_t]),
    "eg2_kfd_lane_ready": (C.c_int, [C.c_void_p, C.c_uint, C.c_char_p, C.c_size_t]),
    "ei_gemma2_kfd_batch": (C.c_bool, [C.c_void_p, _i32, C.POINTER(C.c_size_t), C.c_size_t, _f, C.c_char_p,
                                       C.c_size_t]),
}

_lib = None


def lib():
    """The loaded library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `make -C {HERE}`")
        handle = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


class HipError(RuntimeError):
    pass


def check(code, what):
    if code != 0:
        raise HipError(f"{what}: {lib().eg2_hip_error_string(code).decode()} ({code})")


def synth_gguf(path, seed=0, n_layer=24, dense_head=True, weight_std=0.02, embed_std=0.02, norm_std=0.1,
               rope_base_full=10000.0, rope_base_swa=10000.0, sliding_window=0, sliding_window_pattern=6,
               threads=8):
    """Writes a synthetic gemma-embedding GGUF (see eg2_synth_write_gguf)."""
    cfg = SynthConfig(seed, n_layer, 1 if dense_head else 0, weight_std, embed_std, norm_std, rope_base_full,
                      rope_base_swa, sliding_window, sliding_window_pattern, threads)
    err = C.create_string_buffer(512)
    if lib().eg2_synth_write_gguf(os.fsencode(path), C.byref(cfg), err, 512) != 0:
        raise HipError("synthetic GGUF: " + err.value.decode())


class Gguf:
    """A GGUF file parsed into the engine's ei_gguf layout."""

    def __init__(self, path):
        self.g = EiGguf()
        err = C.create_string_buffer(512)
        if lib().eg2_gguf_open(os.fsencode(path), C.byref(self.g), err, 512) != 0:
            raise HipError(err.value.decode())

    def close(self):
        if self.g is not None:
            lib().eg2_gguf_close(C.byref(self.g))
            self.g = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def validate_gguf(gguf):
    """eg2_kfd_validate_gguf on an open Gguf: None, or the rejection message."""
    err = C.create_string_buffer(512)
    if lib().eg2_kfd_validate_gguf(C.byref(gguf.g), err, 512):
        return None
    return err.value.decode()


class Tokenizer:
    """eg2_tokenizer over the tokenizer.ggml.* keys of a GGUF file."""

    def __init__(self, gguf_path):
        self.gguf = Gguf(gguf_path)
        err = C.create_string_buffer(512)
        self.tok = lib().eg2_tokenizer_create(C.byref(self.gguf.g), err, 512)
        if not self.tok:
            raise HipError(err.value.decode())

    def encode(self, text, add_special=True, parse_special=False):
        """Token ids of `text` (bytes or str) as an int32 array."""
        import numpy as np

        b = text.encode() if isinstance(text, str) else bytes(text)
        n = lib().eg2_tokenize(self.tok, b, len(b), add_special, parse_special, None, 0)
        ids = np.zeros(max(n, 1), np.int32)
        lib().eg2_tokenize(self.tok, b, len(b), add_special, parse_special, ids.ctypes.data_as(_i32), n)
        return ids[:n]

    def encode_batch(self, texts, add_special=True, parse_special=False, threads=0):
        """(ids, offsets) of several texts packed back to back."""
        import numpy as np

        bs = [t.encode() if isinstance(t, str) else bytes(t) for t in texts]
        toffs = (C.c_size_t * (len(bs) + 1))(*np.concatenate([[0], np.cumsum([len(b) for b in bs])]).astype(int))
        joined = b"".join(bs)
        cap = 4 * len(joined) + 4 * len(bs) + 16
        ids = np.zeros(cap, np.int32)
        ioffs = (C.c_size_t * (len(bs) + 1))()
        n = lib().eg2_tokenize_batch(self.tok, joined, toffs, len(bs), add_special, parse_special,
                                     ids.ctypes.data_as(_i32), cap, ioffs, threads)
        if n == (1 << 64) - 1:
            raise HipError("token capacity exceeded")
        return ids[:n], np.array(list(ioffs), np.int64)

    def text_to_id(self, text):
        b = text.encode() if isinstance(text, str) else bytes(text)
        return lib().eg2_tokenizer_text_to_id(self.tok, b, len(b))

    def close(self):
        if getattr(self, "tok", None):
            lib().eg2_tokenizer_free(self.tok)
            self.tok = None
        if getattr(self, "gguf", None):
            self.gguf.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Encoder:
    """ei_gemma2_kfd_create / _batch / _free over a GGUF file."""

    def __init__(self, gguf_path):
        self.gguf = Gguf(gguf_path)
        err = C.create_string_buffer(1024)
        self.ctx = lib().ei_gemma2_kfd_create(C.byref(self.gguf.g), err, 1024)
        if not self.ctx:
            raise HipError(err.value.decode())

    def batch(self, ids, offsets):
        """ids: int32 array of offsets[-1] tokens; offsets: batch+1 sizes.
        Returns float32 [batch, 768] (numpy)."""
        import numpy as np

        ids = np.ascontiguousarray(ids, dtype=np.int32)
        offs = (C.c_size_t * len(offsets))(*[int(o) for o in offsets])
        batch = len(offsets) - 1
        out = np.zeros((max(batch, 1), N_EMBD), dtype=np.float32)
        err = C.create_string_buffer(1024)
        ok = lib().ei_gemma2_kfd_batch(self.ctx, ids.ctypes.data_as(_i32), offs, batch,
                                       out.ctypes.data_as(_f), err, 1024)
        if not ok:
            raise HipError(err.value.decode())
        return out[:batch]

    @property
    def lanes(self):
        """Waves the context keeps in flight (eg2_kfd_lanes)."""
        return lib().eg2_kfd_lanes(self.ctx)

    def stage(self, ids, offsets, lane=0):
        """Uploads one wave to a lane (eg2_kfd_stage_lane); launch()/collect()
        with the same lane then run it."""
        import numpy as np

        if not hasattr(self, "_staged"):
            self._staged = {}
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        offs = (C.c_size_t * len(offsets))(*[int(o) for o in offsets])
        batch = len(offsets) - 1
        err = C.create_string_buffer(1024)
        if not lib().eg2_kfd_stage_lane(self.ctx, lane, ids.ctypes.data_as(_i32), offs, batch, err, 1024):
            raise HipError(err.value.decode())
        self._staged[lane] = batch

    def launch(self, repeats=1, lane=0):
        err = C.create_string_buffer(1024)
        if not lib().eg2_kfd_launch_lane(self.ctx, lane, repeats, err, 1024):
            raise HipError(err.value.decode())

    def ready(self, lane=0):
        """eg2_kfd_lane_ready: True once the lane's enqueued work is done,
        False while it runs (never waits)."""
        err = C.create_string_buffer(1024)
        r = lib().eg2_kfd_lane_ready(self.ctx, lane, err, 1024)
        if r < 0:
            raise HipError(err.value.decode())
        return bool(r)

    def collect(self, lane=0):
        import numpy as np

        out = np.zeros((self._staged[lane], N_EMBD), dtype=np.float32)
        err = C.create_string_buffer(1024)
        if not lib().eg2_kfd_collect_lane(self.ctx, lane, out.ctypes.data_as(_f), err, 1024):
            raise HipError(err.value.decode())
        return out

    def stream(self, ids, text_offsets, dims, cfg=None):
        """eg2_stream_embed: texts ids[text_offsets[i]:text_offsets[i+1]] with
        output widths dims[i], packed into waves by the batcher's rules.
        Returns (float32 [n, 768] with zeros past dims[i], wave count)."""
        import numpy as np

        ids = np.ascontiguousarray(ids, dtype=np.int32)
        n = len(text_offsets) - 1
        offs = (C.c_size_t * (n + 1))(*[int(o) for o in text_offsets])
        d = (C.c_uint * n)(*[int(x) for x in dims])
        cfg = cfg or batch_config()
        out = np.zeros((n, N_EMBD), dtype=np.float32)
        waves = C.c_size_t(0)
        err = C.create_string_buffer(1024)
        if not lib().eg2_stream_embed(self.ctx, ids.ctypes.data_as(_i32), offs, n, d, C.byref(cfg),
                                      out.ctypes.data_as(_f), C.byref(waves), err, 1024):
            raise HipError(err.value.decode())
        return out, waves.value

    def close(self):
        if getattr(self, "ctx", None):
            lib().ei_gemma2_kfd_free(self.ctx)
            self.ctx = None
        if getattr(self, "gguf", None) is not None:
            self.gguf.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def batch_config(**overrides):
    """The launcher's batching settings (eg2_batch_config_default), with overrides."""
    cfg = BatchConfig()
    lib().eg2_batch_config_default(C.byref(cfg))
    for k, v in overrides.items():
        setattr(cfg, k, v)
    return cfg


def pack_waves(lengths, cfg=None):
    """eg2_pack_waves: the list of waves, each a list of sequence indices in
    execution order."""
    n = len(lengths)
    arr = (C.c_size_t * max(n, 1))(*[int(x) for x in lengths])
    order = (C.c_size_t * max(n, 1))()
    ends = (C.c_size_t * max(n, 1))()
    cfg = cfg or batch_config()
    w = lib().eg2_pack_waves(arr, n, C.byref(cfg), order, ends)
    if n and not w:
        raise HipError("eg2_pack_waves rejected its arguments")
    waves, b = [], 0
    for i in range(w):
        waves.append(list(order[b:ends[i]]))
        b = ends[i]
    return waves


def normalize_prefix(embedding, dims):
    """eg2_normalize_prefix on a copy of a 768-float embedding."""
    import numpy as np

    e = np.ascontiguousarray(embedding, dtype=np.float32).copy()
    if not lib().eg2_normalize_prefix(e.ctypes.data_as(_f), dims):
        raise HipError(f"unsupported dims {dims}")
    return e


def rope_table(base, n_pos=N_CTX):
    import numpy as np

    t = np.zeros((n_pos, HEAD_DIM), dtype=np.float32)
    lib().eg2_rope_table(base, n_pos, t.ctypes.data)
    return t


def q8_tile_bytes(rows, k):
    """Bytes of a Q8_0 row-tile buffer (rows rounded up to 32)."""
    return lib().eg2_q8_tile_bytes(rows, k)


def q8_pack_rows(q):
    """int8 [rows, k] -> the row-tile layout (flat int8, padding rows zero)."""
    import numpy as np

    q = np.ascontiguousarray(q, dtype=np.int8)
    rows, k = q.shape
    tiles = np.zeros(q8_tile_bytes(rows, k), dtype=np.int8)
    lib().eg2_q8_pack_rows(q.ctypes.data, rows, k, tiles.ctypes.data)
    return tiles


def q8_unpack_rows(tiles, rows, k):
    """Row-tile bytes -> int8 [rows, k]."""
    import numpy as np

    tiles = np.ascontiguousarray(tiles).view(np.int8)
    assert tiles.size >= q8_tile_bytes(rows, k)
    q = np.zeros((rows, k), dtype=np.int8)
    lib().eg2_q8_unpack_rows(tiles.ctypes.data, rows, k, q.ctypes.data)
    return q


def q8_weight_tiles(blocks_u8, rows, k):
    """GGUF Q8_0 bytes [rows, k] -> the projection GEMM's weight operands
    (wq: int8 row tiles, flat; wd: float32 block scales [k/32, ldw], ldw =
    rows rounded up to 32)."""
    import numpy as np

    src = np.ascontiguousarray(blocks_u8, dtype=np.uint8)
    wq = np.zeros(q8_tile_bytes(rows, k), dtype=np.int8)
    wd = np.zeros((k // 32, (rows + 31) // 32 * 32), dtype=np.float32)
    lib().eg2_q8_weight_tiles(src.ctypes.data, rows, k, wq.ctypes.data, wd.ctypes.data)
    return wq, wd


def q8_geglu_weight_tiles(gate_u8, up_u8, ff, k):
    """GGUF Q8_0 gate and up bytes [ff, k] -> the operands of the fused
    gate|up + GeGLU GEMM (rows interleaved in 32-row groups; wq int8 row
    tiles, flat; wd float32 [k/32, 2 ff])."""
    import numpy as np

    g = np.ascontiguousarray(gate_u8, dtype=np.uint8)
    u = np.ascontiguousarray(up_u8, dtype=np.uint8)
    if g.size != ff * (k // 32) * 34 or u.size != g.size:
        raise ValueError("gate/up must hold ff x k Q8_0 values each")
    wq = np.zeros(q8_tile_bytes(2 * ff, k), dtype=np.int8)
    wd = np.zeros((k // 32, 2 * ff), dtype=np.float32)
    if lib().eg2_q8_geglu_weight_tiles(g.ctypes.data, u.ctypes.data, ff, k, wq.ctypes.data, wd.ctypes.data):
        raise ValueError("ff and k must be multiples of 32")
    return wq, wd


def f32_to_chars(value):
    """eg2_f32_to_chars: the shortest round-trip text of a float32 (None
    for a non-finite value)."""
    buf = C.create_string_buffer(32)
    n = lib().eg2_f32_to_chars(buf, C.c_float(value))
    return buf.raw[:n].decode() if n else None


def base64_f32(values):
    """eg2_base64_f32 of a float32 array."""
    import numpy as np

    v = np.ascontiguousarray(values, dtype=np.float32).ravel()
    buf = C.create_string_buffer(4 * ((4 * v.size + 2) // 3) + 1)
    n = lib().eg2_base64_f32(v.ctypes.data_as(_f), v.size, buf)
    return buf.raw[:n].decode()


def embeddings_response(embeddings, dims, api="ollama", encoding="float", model="", prompt_tokens=0):
    """eg2_embeddings_response: the response body for [n, 768] embeddings
    (normalised to their first `dims` values on a copy)."""
    import numpy as np

    e = np.array(embeddings, dtype=np.float32, copy=True, order="C").reshape(-1, N_EMBD)
    m = model.encode() if isinstance(model, str) else bytes(model)
    cap = lib().eg2_embeddings_response_bound(e.shape[0], dims, len(m))
    buf = C.create_string_buffer(cap + 1)
    n = lib().eg2_embeddings_response(e.ctypes.data_as(_f), e.shape[0], dims, {"ollama": 0, "openai": 1}[api],
                                      {"float": 0, "base64": 1}[encoding], m, len(m), prompt_tokens, buf, cap + 1)
    if n == 0:
        raise ValueError("embedding response failed (dims, non-finite value)")
    return buf.raw[:n].decode()


def attention_capacity(tokens, batch):
    """(items, score floats): eg2_attention_capacity."""
    counts = (C.c_size_t * 2)()
    lib().eg2_attention_capacity(tokens, batch, counts)
    return int(counts[0]), int(counts[1])


def attention_plan(offsets, rows=None):
    """(items uint32 [n, 8], tok uint32 [rows, 4], score floats, score item
    count) of the sequences [offsets[s], offsets[s+1]) (eg2_attention_plan):
    the score items, then the context items; rows defaults to offsets[-1],
    and every row must belong to a sequence."""
    import numpy as np

    offs = (C.c_size_t * len(offsets))(*[int(o) for o in offsets])
    total, batch = int(offsets[-1]), len(offsets) - 1
    rows = total if rows is None else rows
    cap_items, cap_scores = attention_capacity(max(total, 1), max(batch, 1))
    items = np.zeros((cap_items, 8), dtype=np.uint32)
    tok = np.zeros((max(rows, total, 1), 4), dtype=np.uint32)
    counts = (C.c_size_t * 3)()
    rc = lib().eg2_attention_plan(offs, batch, cap_items, cap_scores, items.ctypes.data, tok.ctypes.data, counts)
    if rc != 0:
        raise HipError("attention plan exceeds its capacity")
    return items[:counts[0]], tok[:rows], int(counts[1]), int(counts[2])


class AttentionPlan:
    """The attention plan of a packing on the device (work items, their two
    counts, token records) and its scores scratch."""

    GRID = 1024  # workgroups striding over each item list (the executor's choice)

    def __init__(self, offsets, device, rows=None):
        import numpy as np
        import torch

        items, tok, score_floats, score_items = attention_plan(offsets, rows)
        self.n_items = len(items)
        self.items = torch.from_numpy(np.ascontiguousarray(items).view(np.int32).reshape(-1).copy()
                                      if len(items) else np.zeros(8, np.int32)).to(device)
        self.count = torch.tensor([score_items, len(items) - score_items], dtype=torch.int32, device=device)
        self.tok = torch.from_numpy(np.ascontiguousarray(tok).view(np.int32).reshape(-1).copy()).to(device)
        self.scores = torch.zeros(max(1, score_floats), dtype=torch.float32, device=device)
        self.rows = tok.shape[0]
        self.longest = max(int(offsets[i + 1]) - int(offsets[i]) for i in range(len(offsets) - 1))


class ops:
    """Operator entry points on torch device tensors (current torch stream)."""

    @staticmethod
    def _stream():
        import torch

        return C.c_void_p(torch.cuda.current_stream().cuda_stream)

    @staticmethod
    def _p(t):
        return C.c_void_p(t.data_ptr()) if t is not None else None

    @classmethod
    def embed_norm_quant(cls, table, ids, embed_scale, norm_w, eps, x, xq, xd):
        check(lib().eg2_hip_embed_norm_quant(cls._p(table), cls._p(ids), ids.numel(), embed_scale, cls._p(norm_w),
                                             eps, cls._p(x), cls._p(xq), cls._p(xd), cls._stream()),
              "embed_norm_quant")

    @classmethod
    def residual_norm_quant(cls, x, h, post_w, next_w, eps, xq, xd):
        check(lib().eg2_hip_residual_norm_quant(cls._p(x), cls._p(h), cls._p(post_w), cls._p(next_w), eps,
                                                cls._p(xq), cls._p(xd), x.shape[0], cls._stream()),
              "residual_norm_quant")

    @classmethod
    def qk_norm_rope(cls, qkv, q_w, k_w, table, pos, eps, out):
        """Rows [q0 q1 q2 | k | v] of qkv normalised / rotated into out (may be qkv)."""
        check(lib().eg2_hip_qk_norm_rope(cls._p(qkv), cls._p(q_w), cls._p(k_w), cls._p(table), cls._p(pos), eps,
                                         cls._p(out), qkv.shape[0], cls._stream()), "qk_norm_rope")

    @classmethod
    def gemm_q8_qkv_rope(cls, xq, xd, wq, wd, n, q_w, k_w, table, pos, eps, out):
        """The QKV projection of n rows (xq/xd as for gemm_q8, weights of the
        [q|k|v] concatenation) followed by qk_norm_rope, in one kernel, into
        out [n, 1280]."""
        check(lib().eg2_hip_gemm_q8_qkv_rope(cls._p(xq), cls._p(xd), xd.shape[1], cls._p(wq), cls._p(wd),
                                             wd.shape[1], n, 32 * xd.shape[0], cls._p(q_w), cls._p(k_w),
                                             cls._p(table), cls._p(pos), eps, cls._p(out), cls._stream()),
              "gemm_q8_qkv_rope")

    @classmethod
    def attention(cls, qkv, offsets, window, cq, cd):
        """Packed attention over sequences [offsets[s], offsets[s+1]) of the
        rows [q0 q1 q2 | k | v] of qkv (rows a multiple of 4 covered by the
        sequences), the context quantized into cq / cd."""
        import torch

        plan = AttentionPlan(offsets, qkv.device, qkv.shape[0])
        cls.attention_planned(qkv, plan, window, cq, cd)
        torch.cuda.current_stream().synchronize()  # keeps the plan alive until the kernels ran

    @classmethod
    def attention_planned(cls, qkv, plan, window, cq, cd, longest=None):
        """attention() with a prebuilt AttentionPlan (no host work, no sync);
        longest overrides the plan's longest sequence (0 = the softmax form
        for any length)."""
        check(lib().eg2_hip_attention(cls._p(qkv), cls._p(plan.items), cls._p(plan.count), plan.GRID,
                                      cls._p(plan.tok), window, qkv.shape[0],
                                      plan.longest if longest is None else longest, cls._p(plan.scores),
                                      cls._p(cq), cls._p(cd), cls._stream()), "attention")

    @classmethod
    def attention_stage(cls, stage, qkv, plan, window, cq=None, cd=None, longest=None):
        """One of attention_planned's three kernels stages ("scores",
        "softmax", "context"), for timing them one by one."""
        longest = plan.longest if longest is None else longest
        L = lib()
        if stage == "scores":
            rc = L.eg2_hip_attention_scores(cls._p(qkv), cls._p(plan.items), cls._p(plan.count), plan.GRID, window,
                                            qkv.shape[0], cls._p(plan.scores), cls._stream())
        elif stage == "softmax":
            rc = L.eg2_hip_attention_softmax(cls._p(plan.tok), window, qkv.shape[0], longest, cls._p(plan.scores),
                                             cls._stream())
        elif stage == "context":
            rc = L.eg2_hip_attention_context(cls._p(qkv), cls._p(plan.items), cls._p(plan.count), plan.GRID, window,
                                             qkv.shape[0], cls._p(plan.scores), cls._p(cq), cls._p(cd),
                                             cls._stream())
        else:
            raise ValueError(stage)
        check(rc, "attention_" + stage)

    STATIC_ROWS, STATIC_BATCH = 2048, 2048  # EG2_ATTENTION_STATIC_ROWS / _BATCH

    @classmethod
    def attention_static(cls, qkv, offsets_d, window, cq, cd):
        """attention() through the allocation-free entry point: offsets_d is
        a device uint32/int32 tensor of the batch + 1 sequence bounds; the
        plan is built on the device into the library's static array."""
        rows, batch = qkv.shape[0], offsets_d.numel() - 1
        if rows > cls.STATIC_ROWS or batch > cls.STATIC_BATCH or batch < 1 or rows % 4:
            raise ValueError(f"attention_static: rows {rows} (at most {cls.STATIC_ROWS}, a multiple of 4) and "
                             f"batch {batch} (1 to {cls.STATIC_BATCH}) exceed the static scratch's limits")
        check(lib().eg2_hip_attention_static(cls._p(qkv), cls._p(offsets_d), batch, window, rows, cls._p(cq),
                                             cls._p(cd), cls._stream()), "attention_static")

    @classmethod
    def gelu_quant(cls, gu, gq, gd):
        check(lib().eg2_hip_gelu_quant(cls._p(gu), cls._p(gq), cls._p(gd), gu.shape[0], cls._stream()),
              "gelu_quant")

    @classmethod
    def quantize_rows(cls, x, q, d):
        check(lib().eg2_hip_quantize_rows(cls._p(x), x.shape[1], cls._p(q), cls._p(d), x.shape[0], cls._stream()),
              "quantize_rows")

    @classmethod
    def rms_norm_rows(cls, x, w, eps):
        check(lib().eg2_hip_rms_norm_rows(cls._p(x), cls._p(w), eps, x.shape[0], cls._stream()), "rms_norm_rows")

    @classmethod
    def pool_l2(cls, x, offsets, out):
        check(lib().eg2_hip_pool_l2(cls._p(x), cls._p(offsets), cls._p(out), out.shape[0], cls._stream()),
              "pool_l2")

    @classmethod
    def pool_mean(cls, x, offsets, out):
        check(lib().eg2_hip_pool_mean(cls._p(x), cls._p(offsets), cls._p(out), out.shape[0], cls._stream()),
              "pool_mean")

    @classmethod
    def l2_prefix(cls, x, dims):
        check(lib().eg2_hip_l2_prefix(cls._p(x), x.shape[1], dims, x.shape[0], cls._stream()), "l2_prefix")

    @classmethod
    def op(cls, name, record, grid, block):
        """Launches operator `name` (include/eg2_ops.h) with a record from
        this module; `grid` is a workgroup count or an (x, y) pair."""
        gx, gy = (grid, 1) if isinstance(grid, int) else grid
        check(lib().eg2_op_launch(name.encode(), C.byref(record), C.sizeof(record), gx, gy, block, cls._stream()),
              name)

    @classmethod
    def gemm_q8(cls, xq, xd, wq, wd, y, m=None):
        """y[:, :m] = xq . W^T: xq int8 row tiles of y.shape[0] rows with the
        activation scales xd [k/32, ldx]; (wq, wd) the weights from
        q8_weight_tiles (m defaults to y's width)."""
        n = y.shape[0]
        k = 32 * xd.shape[0]
        m = y.shape[1] if m is None else m
        check(lib().eg2_hip_gemm_q8(cls._p(xq), cls._p(xd), xd.shape[1], cls._p(wq), cls._p(wd), wd.shape[1],
                                    cls._p(y), n, m, k, y.shape[1], cls._stream()), "gemm_q8")

    @classmethod
    def gemm_q8_geglu(cls, xq, xd, wq, wd, gq, gd, n):
        """gq/gd = Q8_0 of gelu(gate) * up for n rows of xq (int8 row tiles,
        scales xd [k/32, ldx]); (wq, wd) from q8_geglu_weight_tiles; gd is
        [ff/32, ldg] and gq the row tiles of ff values per row."""
        k = 32 * xd.shape[0]
        ff = 32 * gd.shape[0]
        check(lib().eg2_hip_gemm_q8_geglu(cls._p(xq), cls._p(xd), xd.shape[1], cls._p(wq), cls._p(wd), wd.shape[1],
                                          cls._p(gq), cls._p(gd), gd.shape[1], n, ff, k, cls._stream()),
              "gemm_q8_geglu")
