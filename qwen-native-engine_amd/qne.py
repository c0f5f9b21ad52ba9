"""Python mirror of the reference's decoder API (kernels/src/model.rs `Model`) over libqne.so.

Same method names, argument meaning and error behaviour as the Rust API: every failure raises
QneError carrying the library's message and code (the reference returns anyhow errors with the same
messages). The library is the product; this module only marshals arguments. It refuses to run
without the built HIP library: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libqne.so"

OK, EINVAL, ECONTEXT, ENOSNAPSHOT, EDEVICE, EFORMAT = 0, -1, -2, -3, -4, -5
MAT_F16, MAT_Q4 = 0, 1
EPI_STORE, EPI_ACCUMULATE, EPI_SWIGLU = 0, 1, 2
MAX_CONTEXT = 4096  # shaders::MAX_CONTEXT (kernels/src/shaders.rs:34), the default capacity

_lib = None


class QneError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


def load_library(path: str | os.PathLike | None = None):
    """Loads libqne.so (built by `make -C qwen-native-engine_amd`), or the build named by the
    QNE_LIBRARY environment variable (the sanitizer build, for instance)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else Path(os.environ.get("QNE_LIBRARY") or LIB_PATH)
    if not p.exists():
        raise QneError(EDEVICE, f"{p} is not built; run make -C {HERE}")
    lib = ctypes.CDLL(str(p))
    c_p, c_sz, c_u32, c_i, c_f = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_int, ctypes.c_float
    sigs = {
        "qne_last_error": ([], ctypes.c_char_p),
        "qne_model_load": ([ctypes.c_char_p, c_sz, c_p, c_sz, ctypes.c_char_p, c_i, ctypes.POINTER(c_p)], c_i),
        "qne_model_free": ([c_p], c_i),
        "qne_reset": ([c_p], c_i),
        "qne_prefill": ([c_p, c_p, c_sz], c_i),
        "qne_prefill_chunk": ([c_p, c_p, c_sz, c_u32, c_i], c_i),
        "qne_logits": ([c_p, c_p, c_sz], c_i),
        "qne_step": ([c_p, c_u32, c_u32, c_p, c_sz], c_i),
        "qne_snapshot": ([c_p], c_i),
        "qne_restore": ([c_p], c_i),
        "qne_last_token": ([c_p, ctypes.POINTER(c_u32), ctypes.POINTER(c_u32)], c_i),
        "qne_decode": ([c_p, c_sz, c_u32, c_p, c_sz, c_p, c_sz, ctypes.POINTER(c_sz)], c_i),
        "qne_decode_ids": ([c_p, c_sz, c_u32, c_p, c_sz, c_p, c_sz, ctypes.POINTER(c_sz)], c_i),
        "qne_dispatches_per_token": ([c_p, ctypes.POINTER(c_sz)], c_i),
        "qne_adapter": ([c_p, ctypes.c_char_p, c_sz], c_i),
        "qne_vocab": ([c_p, ctypes.POINTER(c_u32)], c_i),
        "qne_max_context": ([c_p, ctypes.POINTER(c_u32)], c_i),
        "qne_profile_token": ([c_p, ctypes.POINTER(ctypes.c_double)], c_i),
        "qne_profile_token_json": ([c_p, ctypes.c_char_p, c_sz], c_i),
        "qne_last_decode_timing": ([c_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(c_sz)], c_i),
        "qne_gemv": ([c_i, c_p, c_p, c_i, c_i, c_i, c_p, c_p, c_f, c_p, c_i, c_p], c_i),
        "qne_pack_sz_q4g": ([c_p, c_p, c_sz, c_p], c_i),
        "qne_gdn_step": ([c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i, c_i, c_p], c_i),
        "qne_gdn_prefill_chunked": ([c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i, c_i, c_i, c_p], c_i),
        "qne_paged_attn_decode": ([c_p, c_p, c_p, c_p, c_p, c_p, c_i, c_p, c_p, c_i, c_i, c_i, c_p], c_i),
        "qne_paged_attn_decode_noalloc": ([c_p, c_p, c_p, c_p, c_p, c_p, c_i, c_p, c_p, c_i, c_i, c_i, c_p], c_i),
        "qne_gemm": ([c_i, c_p, c_p, c_i, c_i, c_i, c_p, c_i, c_i, c_p, c_f, c_p, c_i, c_i, c_p], c_i),
        "qne_batch_create": ([c_p, c_u32, c_u32, ctypes.POINTER(c_p)], c_i),
        "qne_batch_free": ([c_p], c_i),
        "qne_batch_admit": ([c_p, c_u32], c_i),
        "qne_batch_reset_row": ([c_p, c_u32, c_u32], c_i),
        "qne_batch_copy_row": ([c_p, c_u32, c_p, c_u32], c_i),
        "qne_batch_row_state": ([c_p, c_u32, c_p, c_p], c_i),
        "qne_batch_step": ([c_p, c_u32, c_p, c_p, c_p, c_sz], c_i),
        "qne_batch_decode": ([c_p, c_u32, c_u32, c_p, c_sz], c_i),
        "qne_batch_fill_synthetic": ([c_p, c_u32, c_p, ctypes.c_uint64], c_i),
        "qne_batch_last_decode_timing": ([c_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(c_sz)], c_i),
        "qne_synth_normal_f32": ([ctypes.c_uint64, ctypes.c_uint64, c_sz, c_f, c_p], c_i),
        "qne_synth_normal_f16": ([ctypes.c_uint64, ctypes.c_uint64, c_sz, c_f, c_p], c_i),
        "qne_quantize_q4g": ([c_p, c_sz, c_sz, c_sz, c_p, c_p, c_p], c_i),
        "qne_step_device": ([c_p, c_u32, c_u32], c_i),
        "qne_logits_device": ([c_p, ctypes.POINTER(c_p)], c_i),
        "qne_stream_read": ([c_p, c_sz, c_p, c_u32, c_p], c_i),
        "qne_noop_dispatch": ([c_p, c_p], c_i),
        "qne_exchange_probe": ([c_p, c_u32, c_u32, c_u32, c_p, ctypes.POINTER(ctypes.c_double)], c_i),
        "qne_sampler_create": ([c_f, c_u32, c_f, ctypes.c_uint64, c_f, c_u32, ctypes.POINTER(c_p)], c_i),
        "qne_sampler_free": ([c_p], c_i),
        "qne_sample": ([c_p, c_p, c_p, c_u32, c_u32, c_f, ctypes.POINTER(c_u32), c_p], c_i),
    }
    for name, (args, res) in sigs.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = res
    if path is None:
        _lib = lib
    return lib


def _check(lib, rc: int):
    if rc != OK:
        raise QneError(rc, lib.qne_last_error().decode("utf-8", "replace"))


def _u32_array(ids):
    a = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32))
    return a, a.ctypes.data_as(ctypes.c_void_p)


class Model:
    """`Model` of kernels/src/model.rs on MI355X. Methods mirror the Rust ones one to one."""

    def __init__(self, handle, lib):
        self._h = handle
        self._lib = lib
        v = ctypes.c_uint32()
        _check(lib, lib.qne_vocab(handle, ctypes.byref(v)))
        self.vocab = v.value
        _check(lib, lib.qne_max_context(handle, ctypes.byref(v)))
        self.max_context = v.value
        buf = ctypes.create_string_buffer(256)
        _check(lib, lib.qne_adapter(handle, buf, 256))
        self.adapter = buf.value.decode()

    @classmethod
    def load(cls, index_json: str, weights, tiles=None, allow_f16: bool = True, options: dict | None = None):
        """Model::load (model.rs:171): validates index.json against the weights, then uploads."""
        import json
        lib = load_library()
        w = np.ascontiguousarray(np.frombuffer(weights, dtype=np.uint8) if not isinstance(weights, np.ndarray)
                                 else weights.view(np.uint8).reshape(-1))
        opts = dict(options or {})
        if tiles is not None:
            opts["tiles"] = tiles
        ij = index_json.encode() if isinstance(index_json, str) else bytes(index_json)
        h = ctypes.c_void_p()
        rc = lib.qne_model_load(ij, len(ij), w.ctypes.data_as(ctypes.c_void_p), w.size,
                                json.dumps(opts).encode() if opts else None, int(allow_f16), ctypes.byref(h))
        _check(lib, rc)
        return cls(h, lib)

    @classmethod
    def load_dir(cls, directory, **kw):
        d = Path(directory)
        return cls.load((d / "index.json").read_text(encoding="utf-8"), np.fromfile(d / "weights.bin", dtype=np.uint8), **kw)

    def close(self):
        if self._h:
            self._lib.qne_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _c(self, rc):
        _check(self._lib, rc)

    def reset(self):
        self._c(self._lib.qne_reset(self._h))

    def prefill(self, ids):
        a, p = _u32_array(ids)
        self._c(self._lib.qne_prefill(self._h, p, a.size))

    def prefill_batched(self, ids):
        self.prefill_from(ids, 0)

    def prefill_from(self, ids, start: int):
        self.prefill_chunk(ids, start, True)

    def prefill_chunk(self, ids, start: int, finish_logits: bool):
        a, p = _u32_array(ids)
        self._c(self._lib.qne_prefill_chunk(self._h, p, a.size, start, int(finish_logits)))

    def logits(self) -> np.ndarray:
        out = np.empty(self.vocab, dtype=np.float32)
        self._c(self._lib.qne_logits(self._h, out.ctypes.data_as(ctypes.c_void_p), out.size))
        return out

    def step(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.vocab, dtype=np.float32)
        self._c(self._lib.qne_step(self._h, token, pos, out.ctypes.data_as(ctypes.c_void_p), out.size))
        return out

    def step_device(self, token: int, pos: int):
        """step without the logits readback; they stay at logits_device() for a Sampler."""
        self._c(self._lib.qne_step_device(self._h, token, pos))

    def logits_device(self) -> int:
        p = ctypes.c_void_p()
        self._c(self._lib.qne_logits_device(self._h, ctypes.byref(p)))
        return p.value

    def snapshot(self):
        self._c(self._lib.qne_snapshot(self._h))

    def restore(self):
        self._c(self._lib.qne_restore(self._h))

    def last_token(self):
        t, p = ctypes.c_uint32(), ctypes.c_uint32()
        self._c(self._lib.qne_last_token(self._h, ctypes.byref(t), ctypes.byref(p)))
        return t.value, p.value

    def decode(self, n: int, window: int = 1, stop=()):
        """Model::decode (model.rs:426-449): a window of more than one step yields u32::MAX
        placeholders, and `stop` is checked against the last value pushed."""
        return self._decode(self._lib.qne_decode, n, window, stop)

    def decode_ids(self, n: int, window: int = 1, stop=()):
        """The same greedy loop returning every id of every window, ending after the first stop id."""
        return self._decode(self._lib.qne_decode_ids, n, window, stop)

    def _decode(self, fn, n, window, stop):
        out = np.zeros(max(n, 1), dtype=np.uint32)
        st, sp = _u32_array(list(stop) if len(stop) else [0])
        ln = ctypes.c_size_t()
        self._c(fn(self._h, n, window, sp, len(stop), out.ctypes.data_as(ctypes.c_void_p), out.size, ctypes.byref(ln)))
        return [int(x) for x in out[:ln.value]]

    def dispatches_per_token(self) -> int:
        v = ctypes.c_size_t()
        self._c(self._lib.qne_dispatches_per_token(self._h, ctypes.byref(v)))
        return v.value

    def profile_token(self) -> float:
        v = ctypes.c_double()
        self._c(self._lib.qne_profile_token(self._h, ctypes.byref(v)))
        return v.value

    def profile_token_detail(self) -> dict:
        """Model::profile_token (model.rs:305) with the per-phase timeline: consumes one greedy token."""
        import json
        buf = ctypes.create_string_buffer(16 << 20)
        self._c(self._lib.qne_profile_token_json(self._h, buf, len(buf)))
        return json.loads(buf.value.decode())

    def profile_labels(self) -> dict:
        """label -> ms for one greedy token, as the reference's profile_token returns."""
        return self.profile_token_detail()["labels"]

    def last_decode_timing(self):
        """(device ms, steps) of the windows of the last decode call (HIP events)."""
        ms, n = ctypes.c_double(), ctypes.c_size_t()
        self._c(self._lib.qne_last_decode_timing(self._h, ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value


class Sampler:
    """src/sampling.rs Sampler over device logits (temperature + top-k + top-p, presence penalty,
    grammar mask): the O(vocab) part on the GPU, the draw on the host in the reference's f32
    arithmetic."""

    def __init__(self, vocab: int, temperature: float = 0.6, top_k: int = 20, top_p: float = 0.95, seed: int = 42,
                 presence_penalty: float = 0.0, lib=None):
        self._lib = lib or load_library()
        h = ctypes.c_void_p()
        _check(self._lib, self._lib.qne_sampler_create(temperature, top_k, top_p, seed, presence_penalty, vocab,
                                                       ctypes.byref(h)))
        self._h = h
        self.vocab = vocab

    def close(self):
        if self._h:
            self._lib.qne_sampler_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def sample(self, logits_ptr: int, mask=None, mask_len: int = 0, bias_token: int = 0xFFFFFFFF,
               bias: float = 0.0, stream: int = 0) -> int:
        """Sampler::try_sample over `vocab` logits at device address logits_ptr. mask: a uint32
        bitset (bit i%32 of word i/32 allows token i) covering mask_len tokens, or None."""
        t = ctypes.c_uint32()
        if mask is not None:
            m = np.ascontiguousarray(np.asarray(mask, dtype=np.uint32))
            mp = m.ctypes.data_as(ctypes.c_void_p)
        else:
            m, mp, mask_len = None, None, 0
        _check(self._lib, self._lib.qne_sample(self._h, logits_ptr, mp, mask_len, bias_token, bias, ctypes.byref(t),
                                               stream))
        return t.value


class Batch:
    """Batched continuous decode over one model's weights: rows 0..n-1 each hold a sequence with its
    own KV cache and recurrent state, and every step advances all of them by one token."""

    def __init__(self, model: Model, max_rows: int, max_context: int):
        self._lib = model._lib
        self._model = model  # the weights must outlive the batch
        h = ctypes.c_void_p()
        _check(self._lib, self._lib.qne_batch_create(model._h, max_rows, max_context, ctypes.byref(h)))
        self._h = h
        self.max_rows = max_rows
        self.vocab = model.vocab

    def close(self):
        if self._h:
            self._lib.qne_batch_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _c(self, rc):
        _check(self._lib, rc)

    def admit(self, row: int):
        """Row `row` takes over the model's current sequence (state, next token and position)."""
        self._c(self._lib.qne_batch_admit(self._h, row))

    def copy_row(self, row: int, src: "Batch", src_row: int):
        """Row `row` takes over row `src_row` of `src` (a batch over the same model)."""
        self._c(self._lib.qne_batch_copy_row(self._h, row, src._h, src_row))

    def reset_row(self, row: int, token: int):
        self._c(self._lib.qne_batch_reset_row(self._h, row, token))

    def row_state(self, n: int):
        t = np.zeros(n, dtype=np.uint32)
        p = np.zeros(n, dtype=np.uint32)
        self._c(self._lib.qne_batch_row_state(self._h, n, t.ctypes.data_as(ctypes.c_void_p),
                                               p.ctypes.data_as(ctypes.c_void_p)))
        return t, p

    def step(self, n: int, tokens=None, logits: bool = False):
        """One step of rows 0..n-1; returns (greedy picks, logits [n][vocab] or None)."""
        nxt = np.zeros(n, dtype=np.uint32)
        tp = None
        if tokens is not None:
            ta, tp = _u32_array(tokens)
            assert ta.size == n
        lg = np.zeros((n, self.vocab), dtype=np.float32) if logits else None
        self._c(self._lib.qne_batch_step(self._h, n, tp, nxt.ctypes.data_as(ctypes.c_void_p),
                                         lg.ctypes.data_as(ctypes.c_void_p) if logits else None,
                                         lg.size if logits else 0))
        return nxt, lg

    def decode(self, n: int, steps: int):
        """`steps` greedy steps of rows 0..n-1 on the device; returns ids [steps][n]."""
        out = np.zeros((max(steps, 1), n), dtype=np.uint32)
        self._c(self._lib.qne_batch_decode(self._h, n, steps, out.ctypes.data_as(ctypes.c_void_p), out.size))
        return out[:steps]

    def fill_synthetic(self, ctx, seed: int = 0):
        ca, cp = _u32_array(ctx)
        self._c(self._lib.qne_batch_fill_synthetic(self._h, ca.size, cp, seed))

    def last_decode_timing(self):
        ms, n = ctypes.c_double(), ctypes.c_size_t()
        self._c(self._lib.qne_batch_last_decode_timing(self._h, ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value


# ---- kernel-level entry points on device pointers (ints) ----

def gemm(kind, w, sz, rows, k, group, x, x_stride, m, y, y_stride, epilogue=EPI_STORE, norm=0, eps=1e-6, stream=0):
    lib = load_library()
    _check(lib, lib.qne_gemm(kind, w, sz or None, rows, k, group, x, x_stride, m, norm or None, eps, y, y_stride,
                             epilogue, stream or None))



def gemv(kind, w, sz, rows, k, group, x, y, epilogue=EPI_STORE, norm=0, eps=1e-6, stream=0):
    lib = load_library()
    _check(lib, lib.qne_gemv(kind, w, sz or None, rows, k, group, x, norm or None, eps, y, epilogue, stream or None))


def gdn_step(q, k, v, beta, g, state, out, batch, heads, stream=0):
    lib = load_library()
    _check(lib, lib.qne_gdn_step(q, k, v, beta, g, state, out, batch, heads, stream or None))


def gdn_prefill_chunked(q, k, v, beta, g, state, out, batch, tokens, heads, stream=0):
    lib = load_library()
    _check(lib, lib.qne_gdn_prefill_chunked(q, k, v, beta, g, state, out, batch, tokens, heads, stream or None))


def paged_attn_decode(q, k_new, v_new, k_pool, v_pool, block_table, max_blocks, ctx, out, batch, nq, nkv, stream=0):
    lib = load_library()
    _check(lib, lib.qne_paged_attn_decode(q, k_new, v_new, k_pool, v_pool, block_table, max_blocks, ctx, out, batch,
                                          nq, nkv, stream or None))


def paged_attn_decode_noalloc(q, k_new, v_new, k_pool, v_pool, block_table, max_blocks, ctx, out, batch, nq, nkv,
                              stream=0):
    """paged_attn_decode with its split partials in the library's fixed per-GPU array (no allocation)."""
    lib = load_library()
    _check(lib, lib.qne_paged_attn_decode_noalloc(q, k_new, v_new, k_pool, v_pool, block_table, max_blocks, ctx, out,
                                                  batch, nq, nkv, stream or None))
