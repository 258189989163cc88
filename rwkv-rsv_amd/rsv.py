"""Python binding of the MI355X RWKV-7 library (ctypes over the C-ABI).

Mirrors the reference's public API (src/gpu_model.rs:3685-3913):

    bundle = ModelBuilder(path).build()
    logits = bundle.infer_seq(tokens)          # prefill
    logits = bundle.infer_tokens(tokens)       # token-by-token decode
    toks   = bundle.infer_argmax_selfloop(seed, n)
    toks   = bundle.infer_sample_selfloop(seed, n, SamplerParams(...))
    data   = bundle.state_back(); bundle.state_load(data); bundle.reset()

plus the batch API of GpuModel (create_batch_state, forward_seq_batch,
sample/argmax self-loops over a batch State).  `Backend` exposes the
op-level C-ABI of librsv_hip.so (the ComputeBackend surface) for tests.

Everything runs on the HIP libraries built in-tree under _build/; importing
this module fails loudly when they are missing -- there is no CPU fallback.
"""
import ctypes
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
BUILD = os.path.join(HERE, "_build")
HIP_LIB = os.path.join(BUILD, "librsv_hip.so")
HOST_LIB = os.path.join(BUILD, "librsv_host.so")

F32, F16, U32 = 0, 1, 2
NONE = 0xFFFFFFFF


class RsvError(RuntimeError):
    pass


INCLUDE = os.path.join(os.path.dirname(HERE), "include")


class Int8Handle(ctypes.Structure):
    """rsv_int8 (Int8Handle, backend.rs:36-44)."""
    _fields_ = [("idx", ctypes.c_uint32), ("sz", ctypes.c_uint32), ("m", ctypes.c_uint64), ("k", ctypes.c_uint64)]


class GemvJob(ctypes.Structure):
    """rsv_gemv_job (include/rsv_hip.h)."""
    _fields_ = [("w16", ctypes.c_uint32), ("w8", ctypes.POINTER(Int8Handle)), ("m", ctypes.c_uint64),
                ("k", ctypes.c_uint64), ("x", ctypes.c_uint32), ("y", ctypes.c_uint32), ("prologue", ctypes.c_int),
                ("epilogue", ctypes.c_int), ("xmul", ctypes.c_uint32), ("p0", ctypes.c_uint32),
                ("p1", ctypes.c_uint32), ("scale", ctypes.c_uint32), ("gamma", ctypes.c_uint32),
                ("beta", ctypes.c_uint32), ("prev", ctypes.c_uint32), ("coef", ctypes.c_uint32),
                ("lnout", ctypes.c_uint32), ("gn_eps", ctypes.c_float)]


class MmJob(ctypes.Structure):
    """rsv_mm_job (include/rsv_hip.h)."""
    _fields_ = [("w16", ctypes.c_uint32), ("w8", ctypes.POINTER(Int8Handle)), ("n", ctypes.c_uint64),
                ("k", ctypes.c_uint64), ("x", ctypes.c_uint32), ("y", ctypes.c_uint32), ("y2", ctypes.c_uint32),
                ("epilogue", ctypes.c_int), ("bias", ctypes.c_uint32), ("aux", ctypes.c_uint32),
                ("scale", ctypes.c_uint32), ("tiled", ctypes.c_int)]


def _ctype(decl):
    d = decl.replace("const", "").strip()
    ptr = d.count("*")
    base = d.replace("*", " ").split()[0]
    scalars = {"uint32_t": ctypes.c_uint32, "uint64_t": ctypes.c_uint64, "float": ctypes.c_float,
               "int": ctypes.c_int, "size_t": ctypes.c_size_t, "uint16_t": ctypes.c_uint16}
    if ptr == 0:
        return scalars[base]
    if ptr == 2 or base in ("void", "rsv_ctx", "rsv_bundle", "rsv_state"):
        return ctypes.c_void_p if ptr == 1 else ctypes.POINTER(ctypes.c_void_p)
    if base == "char":
        return ctypes.c_char_p
    if base == "rsv_int8":
        return ctypes.POINTER(Int8Handle)
    if base in ("rsv_model_info", "rsv_sampler_params", "rsv_gemv_job", "rsv_mm_job", "rsv_serve_step",
                "rsv_wkv_lora"):
        return ctypes.c_void_p
    return ctypes.POINTER(scalars[base])


def declare(lib, header):
    """Sets argtypes/restype of every prototype in an include/*.h file and
    returns the declared names (used by the export test)."""
    import re
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    names = []
    for m in re.finditer(r"^\s*(int|uint64_t|const char \*|void \*)\s*(rsv_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        ret, name, args = m.group(1).strip(), m.group(2), m.group(3)
        names.append(name)
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        argl = [a.strip() for a in args.split(",") if a.strip() and a.strip() != "void"]
        types = []
        for a in argl:
            decl = a.rsplit(None, 1)[0] if not a.endswith("*") else a
            if "*" in a.split()[-1]:  # "float *out" style: name carries the star
                decl = a.rsplit(None, 1)[0] + " " + "*" * a.split()[-1].count("*")
            types.append(_ctype(decl))
        fn.argtypes = types
        fn.restype = {"int": ctypes.c_int, "uint64_t": ctypes.c_uint64, "const char *": ctypes.c_char_p,
                      "void *": ctypes.c_void_p}[ret]
    return names


def _load():
    for p in (HIP_LIB, HOST_LIB):
        if not os.path.exists(p):
            raise RsvError(f"{p} is not built; run `python __graft_entry__.py build` (or rwkv-rsv_amd/rsv_build.py)")
    hip = ctypes.CDLL(HIP_LIB, mode=ctypes.RTLD_GLOBAL)
    host = ctypes.CDLL(HOST_LIB)
    declare(hip, os.path.join(INCLUDE, "rsv_hip.h"))
    declare(host, os.path.join(INCLUDE, "rsv_host.h"))
    return hip, host


_hip, _host = _load()


def hip_lib():
    return _hip


def host_lib():
    return _host


def _u32p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))


def _f32p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _u64p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64))


def _hchk(rc):
    if rc != 0:
        raise RsvError(_host.rsv_host_last_error().decode())


def _bchk(rc):
    if rc != 0:
        raise RsvError(_hip.rsv_last_error().decode())


class ModelInfo(ctypes.Structure):
    _fields_ = [("n_layer", ctypes.c_uint64), ("n_embd", ctypes.c_uint64), ("n_head", ctypes.c_uint64),
                ("head_size", ctypes.c_uint64), ("vocab", ctypes.c_uint64), ("ffn", ctypes.c_uint64),
                ("w_mid", ctypes.c_uint64), ("a_mid", ctypes.c_uint64), ("v_mid", ctypes.c_uint64),
                ("g_mid", ctypes.c_uint64), ("int8_linears", ctypes.c_int), ("int8_head", ctypes.c_int)]

    @property
    def num_vocab(self):
        return self.vocab


class ServeStep(ctypes.Structure):
    """rsv_serve_step (include/rsv_host.h): one dispatch of serve_ragged."""
    _fields_ = [("prefill_tokens", ctypes.c_uint64), ("decode_tokens", ctypes.c_uint64),
                ("sampled", ctypes.c_uint64), ("ms", ctypes.c_double)]


class _SP(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_uint32), ("top_p", ctypes.c_float),
                ("seed", ctypes.c_uint32), ("repetition_penalty", ctypes.c_float),
                ("frequency_penalty", ctypes.c_float), ("presence_penalty", ctypes.c_float)]


@dataclass
class SamplerParams:
    """SamplerParams (gpu_model.rs:3873-3911); defaults match Default."""
    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    seed: int = 0
    repetition_penalty: float = 1.0
    frequency_penalty: float = 0.0
    presence_penalty: float = 0.0

    def _c(self):
        return _SP(self.temperature, self.top_k, self.top_p, self.seed & 0xFFFFFFFF, self.repetition_penalty,
                   self.frequency_penalty, self.presence_penalty)


def _toks(tokens):
    return np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32).reshape(-1))


class State:
    """A batch State (gpu_model.rs:3920-4105) owned by a Bundle's model."""

    def __init__(self, bundle, handle, batch):
        self._b = bundle
        self._h = handle
        self.batch = batch

    def back(self):
        out = np.empty(self.batch * self._b.state_len, np.float32)
        _hchk(_host.rsv_batch_state_back(self._b._h, self._h, _f32p(out)))
        return out

    def load(self, data):
        d = np.ascontiguousarray(data, dtype=np.float32)
        _hchk(_host.rsv_batch_state_load(self._b._h, self._h, _f32p(d), ctypes.c_uint64(d.size)))

    def slot_back(self, slot):
        out = np.empty(self._b.state_len, np.float32)
        _hchk(_host.rsv_state_slot_back(self._b._h, self._h, ctypes.c_uint64(slot), _f32p(out)))
        return out

    def slot_load(self, slot, data):
        d = np.ascontiguousarray(data, dtype=np.float32)
        _hchk(_host.rsv_state_slot_load(self._b._h, self._h, ctypes.c_uint64(slot), _f32p(d), ctypes.c_uint64(d.size)))

    def reset(self):
        _hchk(_host.rsv_batch_state_reset(self._b._h, self._h))

    def free(self):
        if self._h:
            _host.rsv_state_free(self._b._h, self._h)
            self._h = None


class Bundle:
    """Model + one session State (gpu_model.rs:3705-3860)."""

    def __init__(self, handle):
        self._h = handle
        info = ModelInfo()
        _hchk(_host.rsv_bundle_info(self._h, ctypes.byref(info)))
        self._info = info
        n = ctypes.c_uint64()
        _hchk(_host.rsv_state_len(self._h, ctypes.byref(n)))
        self.state_len = n.value
        self.vocab = info.vocab

    def build_shared(self):
        """GpuModel::build_shared: a second bundle sharing this one's weights."""
        h = ctypes.c_void_p()
        _hchk(_host.rsv_bundle_build_shared(self._h, ctypes.byref(h)))
        return Bundle(h)

    def close(self):
        if self._h:
            _host.rsv_bundle_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self):
        return self._info

    def ctx(self):
        return _host.rsv_bundle_ctx(self._h)

    # ---- single session
    def infer_tokens(self, tokens):
        t = _toks(tokens)
        out = np.empty(self.vocab, np.float32)
        _hchk(_host.rsv_infer_tokens(self._h, _u32p(t), ctypes.c_uint64(t.size), _f32p(out)))
        return out

    def infer_seq(self, tokens):
        t = _toks(tokens)
        out = np.empty(self.vocab, np.float32)
        _hchk(_host.rsv_infer_seq(self._h, _u32p(t), ctypes.c_uint64(t.size), _f32p(out)))
        return out

    def infer_chunked(self, tokens, chunk_size):
        t = _toks(tokens)
        out = np.empty(self.vocab, np.float32)
        _hchk(_host.rsv_infer_chunked(self._h, _u32p(t), ctypes.c_uint64(t.size), ctypes.c_uint64(chunk_size),
                                      _f32p(out)))
        return out

    def infer_full(self, tokens):
        t = _toks(tokens)
        out = np.empty(t.size * self.vocab, np.float32)
        _hchk(_host.rsv_infer_full(self._h, _u32p(t), ctypes.c_uint64(t.size), _f32p(out)))
        return out.reshape(t.size, self.vocab)

    def infer_argmax(self, tokens):
        t = _toks(tokens)
        out = np.zeros(1, np.uint32)
        _hchk(_host.rsv_infer_argmax(self._h, _u32p(t), ctypes.c_uint64(t.size), _u32p(out)))
        return int(out[0])

    def infer_argmax_selfloop(self, seed, n):
        out = np.zeros(n, np.uint32)
        _hchk(_host.rsv_infer_argmax_selfloop(self._h, ctypes.c_uint32(seed), ctypes.c_uint64(n), _u32p(out)))
        return out

    def infer_sample(self, tokens, sp, history=()):
        t = _toks(tokens)
        h = _toks(history) if len(history) else np.zeros(1, np.uint32)
        out = np.zeros(1, np.uint32)
        c = sp._c()
        _hchk(_host.rsv_infer_sample(self._h, _u32p(t), ctypes.c_uint64(t.size), ctypes.byref(c), _u32p(h),
                                     ctypes.c_uint64(len(history)), _u32p(out)))
        return int(out[0])

    def infer_sample_selfloop(self, seed, n, sp):
        out = np.zeros(n, np.uint32)
        c = sp._c()
        _hchk(_host.rsv_infer_sample_selfloop(self._h, ctypes.c_uint32(seed), ctypes.c_uint64(n), ctypes.byref(c),
                                              _u32p(out)))
        return out

    def state_back(self):
        out = np.empty(self.state_len, np.float32)
        _hchk(_host.rsv_state_back(self._h, _f32p(out)))
        return out

    def state_load(self, data):
        d = np.ascontiguousarray(data, dtype=np.float32)
        _hchk(_host.rsv_state_load(self._h, _f32p(d), ctypes.c_uint64(d.size)))

    def reset(self):
        _hchk(_host.rsv_reset(self._h))

    # ---- batch (GpuModel, gpu_model.rs:871-1803)
    def create_batch_state(self, batch):
        h = ctypes.c_void_p()
        _hchk(_host.rsv_create_batch_state(self._h, ctypes.c_uint64(batch), ctypes.byref(h)))
        return State(self, h, batch)

    def set_prefill_chunk(self, rows):
        """Rows per packed prefill chunk (1..12288, default 4096: the reference's packing bound)."""
        _hchk(_host.rsv_set_prefill_chunk(self._h, ctypes.c_uint64(rows)))

    def set_prefill_lanes(self, lanes):
        """Streams of a multi-chunk prefill (1 or 2; 2 overlaps consecutive
        chunks, bit-identical results)."""
        _hchk(_host.rsv_set_prefill_lanes(self._h, ctypes.c_int(lanes)))

    def forward_seq_batch(self, state, prompts, want_logits=False):
        lens = np.array([len(p) for p in prompts], dtype=np.uint64)
        flat = _toks(np.concatenate([np.asarray(p, dtype=np.uint32) for p in prompts]))
        seeds = np.zeros(len(prompts), np.uint32)
        lg = np.empty(len(prompts) * self.vocab, np.float32) if want_logits else None
        _hchk(_host.rsv_forward_seq_batch(self._h, state._h, _u32p(flat), _u64p(lens), _u32p(seeds),
                                          _f32p(lg) if lg is not None else None))
        return (seeds, lg.reshape(len(prompts), self.vocab)) if want_logits else seeds

    def forward_tokens_batch(self, state, tokens):
        t = _toks(tokens)
        out = np.empty(state.batch * self.vocab, np.float32)
        _hchk(_host.rsv_forward_tokens_batch(self._h, state._h, _u32p(t), _f32p(out)))
        return out.reshape(state.batch, self.vocab)

    def argmax_selfloop_batch(self, state, seeds, n):
        s = _toks(seeds)
        out = np.zeros(state.batch * n, np.uint32)
        _hchk(_host.rsv_argmax_selfloop_batch(self._h, state._h, _u32p(s), ctypes.c_uint64(n), _u32p(out)))
        return out.reshape(state.batch, n)

    def argmax_selfloop_batch_timed(self, state, seeds, n):
        s = _toks(seeds)
        out = np.zeros(state.batch * n, np.uint32)
        ms = ctypes.c_float()
        _hchk(_host.rsv_argmax_selfloop_batch_timed(self._h, state._h, _u32p(s), ctypes.c_uint64(n), _u32p(out),
                                                    ctypes.byref(ms)))
        return out.reshape(state.batch, n), ms.value

    def sample_selfloop_batch_timed(self, state, seeds, n, sp):
        s = _toks(seeds)
        out = np.zeros(state.batch * n, np.uint32)
        c = sp._c()
        ms = ctypes.c_float()
        _hchk(_host.rsv_sample_selfloop_batch_timed(self._h, state._h, _u32p(s), ctypes.c_uint64(n), ctypes.byref(c),
                                                    _u32p(out), ctypes.byref(ms)))
        return out.reshape(state.batch, n), ms.value

    def sample_selfloop_batch(self, state, seeds, n, sp):
        s = _toks(seeds)
        out = np.zeros(state.batch * n, np.uint32)
        c = sp._c()
        _hchk(_host.rsv_sample_selfloop_batch(self._h, state._h, _u32p(s), ctypes.c_uint64(n), ctypes.byref(c),
                                              _u32p(out)))
        return out.reshape(state.batch, n)


    def serve_ragged(self, state, prompts, decode_len, sp, seeds, budget=4096, max_steps=None, want_logits=False):
        """Ragged continuous batching over the slots of `state`: slot q
        prefills prompts[q] and samples `decode_len` tokens; every step is one
        packed dispatch of decode tokens plus prompt chunks (`budget` tokens).
        Returns (tokens [batch, decode_len], list of per-step dicts), and with
        want_logits the logits row of every draw [batch, decode_len, vocab]."""
        if len(prompts) != state.batch:
            raise RsvError(f"serve_ragged: {len(prompts)} prompts for {state.batch} slots")
        lens = np.array([len(p) for p in prompts], np.uint64)
        flat = _toks(np.concatenate([np.asarray(p, np.uint32) for p in prompts]))
        sd = _toks(seeds)
        out = np.zeros(state.batch * decode_len, np.uint32)
        if max_steps is None:
            max_steps = int(lens.sum()) + state.batch * decode_len + 16
        steps = (ServeStep * max_steps)()
        n = ctypes.c_uint64()
        c = sp._c()
        args = (self._h, state._h, _u32p(flat), _u64p(lens), ctypes.c_uint64(decode_len), ctypes.byref(c), _u32p(sd),
                ctypes.c_uint64(budget), _u32p(out), ctypes.cast(steps, ctypes.c_void_p), ctypes.c_uint64(max_steps),
                ctypes.byref(n))
        lg = None
        if want_logits:
            lg = np.zeros((state.batch, decode_len, self.vocab), np.float32)
            _hchk(_host.rsv_serve_ragged_logits(*args, lg.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        else:
            _hchk(_host.rsv_serve_ragged(*args))
        recs = [dict(prefill_tokens=steps[i].prefill_tokens, decode_tokens=steps[i].decode_tokens,
                     sampled=steps[i].sampled, ms=steps[i].ms) for i in range(n.value)]
        if want_logits:
            return out.reshape(state.batch, decode_len), recs, lg
        return out.reshape(state.batch, decode_len), recs


class ModelBuilder:
    """ModelBuilder::new(path).build() (gpu_model.rs:3685-3703)."""

    def __init__(self, path, device=0):
        self.path = path
        self.device = device

    def build(self):
        h = ctypes.c_void_p()
        _hchk(_host.rsv_model_build(self.path.encode(), self.device, ctypes.byref(h)))
        return Bundle(h)


class Backend:
    """Op-level access to librsv_hip.so (the ComputeBackend C-ABI)."""

    def __init__(self, device=0):
        self.ctx = ctypes.c_void_p()
        _bchk(_hip.rsv_create(device, ctypes.byref(self.ctx)))
        self._ids = []

    def close(self):
        if self.ctx:
            _hip.rsv_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def call(self, name, *args):
        _bchk(getattr(_hip, name)(self.ctx, *args))

    def tensor(self, data=None, n=None, dtype=F32):
        tid = ctypes.c_uint32()
        if data is not None:
            a = np.asarray(data)
            n = a.size
        _bchk(_hip.rsv_tensor_create(self.ctx, ctypes.c_uint64(n), dtype, ctypes.byref(tid)))
        if data is not None:
            if dtype == U32:
                a = np.ascontiguousarray(a, dtype=np.uint32).reshape(-1)
                _bchk(_hip.rsv_upload_u32(self.ctx, tid, _u32p(a), ctypes.c_uint64(a.size)))
            else:
                a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
                _bchk(_hip.rsv_upload(self.ctx, tid, _f32p(a), ctypes.c_uint64(a.size)))
        return tid.value

    def bytes_tensor(self, raw, n_words):
        """U32 tensor filled with raw bytes (e.g. u8 int8_idx payloads)."""
        tid = self.tensor(n=n_words, dtype=U32)
        b = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
        _bchk(_hip.rsv_upload_bytes(self.ctx, tid, b.ctypes.data_as(ctypes.c_void_p), ctypes.c_uint64(b.size)))
        return tid

    def get(self, tid, n, dtype=F32):
        if dtype == U32:
            out = np.empty(n, np.uint32)
            _bchk(_hip.rsv_download_u32(self.ctx, tid, _u32p(out), ctypes.c_uint64(n)))
        else:
            out = np.empty(n, np.float32)
            _bchk(_hip.rsv_download(self.ctx, tid, _f32p(out), ctypes.c_uint64(n)))
        return out

    def int8(self, idx, sz):
        """rsv_int8 handle from u8 idx [m,k] and u32 sz [m,k/128]."""
        m, k = idx.shape
        h = Int8Handle(self.bytes_tensor(idx, m * k // 4), self.tensor(sz.reshape(-1), dtype=U32), m, k)
        return h

    def sync(self):
        _bchk(_hip.rsv_synchronize(self.ctx))


def u64(v):
    return ctypes.c_uint64(v)


def f32(v):
    return ctypes.c_float(v)
