"""CPU fp32 oracle for the rwkv-rsv RWKV-7 forward step -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker or the reported CPU baseline.  The
product path (librsv_hip.so / librsv_host.so) never calls it.

The arithmetic lives in rsv_oracle.c (a restatement of the reference's
src/model.rs); this file loads a safetensors model the way
Model::from_safetensors does (model.rs:276-346, 534-620): every tensor as
f32, int8 linears dequantised with the restated dequant (model.rs:234-252),
linear and head weights transposed to [in, out], LoRA matrices oriented by
shape.  Files are read with safetensors' numpy loader (no pickle).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "liboracle.so")

# per-layer pointer order of rsv_oracle.c's L_* enum
FIELDS = ["ln1.weight", "ln1.bias", "att.x_r", "att.x_w", "att.x_k", "att.x_v", "att.x_a", "att.x_g",
          "att.w0", "att.a0", "att.v0", "att.w1", "att.w2", "att.a1", "att.a2", "att.v1", "att.v2",
          "att.g1", "att.g2", "att.r_k", "att.k_k", "att.k_a", "att.receptance.weight", "att.key.weight",
          "att.value.weight", "att.output.weight", "att.ln_x.weight", "att.ln_x.bias", "ln2.weight",
          "ln2.bias", "ffn.x_k", "ffn.key.weight", "ffn.value.weight"]

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        f32p = ctypes.POINTER(ctypes.c_float)
        u32p = ctypes.POINTER(ctypes.c_uint32)
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_dequant_int8.argtypes = [u32p, u32p, ctypes.c_int64, ctypes.c_int64, f32p]
        L.orc_layer_norm.argtypes = [f32p, f32p, f32p, ctypes.c_int64, ctypes.c_float, f32p]
        L.orc_group_norm.argtypes = [f32p, f32p, f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_float, f32p]
        L.orc_layer_norm_rows.argtypes = [f32p, f32p, f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_float, f32p]
        L.orc_matvec.argtypes = [f32p, f32p, ctypes.c_int64, ctypes.c_int64, f32p]
        L.orc_l2_norm_groups.argtypes = [f32p, ctypes.c_int64, ctypes.c_int64, f32p]
        L.orc_dplr_update.argtypes = [f32p, f32p, f32p, f32p, f32p, f32p, ctypes.c_int64, ctypes.c_int64]
        L.orc_dplr_matvec.argtypes = [f32p, f32p, ctypes.c_int64, ctypes.c_int64, f32p]
        L.orc_sum_rk_rk.argtypes = [f32p, f32p, f32p, f32p, ctypes.c_int64, ctypes.c_int64, f32p]
        L.orc_argmax.restype = ctypes.c_uint32
        L.orc_argmax.argtypes = [f32p, ctypes.c_int64]
        L.orc_u01.restype = ctypes.c_float
        L.orc_u01.argtypes = [ctypes.c_uint32]
        L.orc_sample.restype = ctypes.c_uint32
        L.orc_sample.argtypes = [f32p, ctypes.c_int64, ctypes.c_float, ctypes.c_uint32, ctypes.c_float,
                                 ctypes.c_uint32, ctypes.c_float, ctypes.c_float, ctypes.c_float, u32p,
                                 ctypes.c_uint32, f32p]
        L.orc_set_threads.argtypes = [ctypes.c_int]
        L.orc_nfields.restype = ctypes.c_int
        L.orc_state_len.restype = ctypes.c_int64
        L.orc_forward.argtypes = [ctypes.c_void_p, u32p, ctypes.c_int64, f32p, f32p]
        assert L.orc_nfields() == len(FIELDS)
        _lib = L
    return _lib


def set_threads(n):
    """Splits the oracle's matvec columns over n threads (bit-identical to one
    thread; a checker speed-up for the 3B tests).  The CPU baseline uses 1."""
    lib().orc_set_threads(int(n))


def fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def up(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))


def f32c(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ------------------------------------------------------------ primitives
def dequant_int8(idx, sz, m, k):
    idx = np.ascontiguousarray(idx).view(np.uint8).reshape(-1)
    w = np.empty(m * k, np.float32)
    idx32 = np.ascontiguousarray(idx).view(np.uint32)
    sz = np.ascontiguousarray(sz, dtype=np.uint32).reshape(-1)
    lib().orc_dequant_int8(up(idx32), up(sz), m, k, fp(w))
    return w.reshape(m, k)


def layer_norm(x, w, b, eps=1e-5):
    x, w, b = f32c(x), f32c(w), f32c(b)
    y = np.empty_like(x)
    lib().orc_layer_norm(fp(x), fp(w), fp(b), x.size, eps, fp(y))
    return y


def group_norm(x, w, b, h, n, eps=64e-5):
    x, w, b = f32c(x), f32c(w), f32c(b)
    y = np.empty_like(x)
    lib().orc_group_norm(fp(x), fp(w), fp(b), h, n, eps, fp(y))
    return y


def matvec(x, w):
    """y = x @ W with W [in, out] (model.rs:700-713)."""
    x, w = f32c(x), f32c(w)
    y = np.empty(w.shape[1], np.float32)
    lib().orc_matvec(fp(x), fp(w), w.shape[0], w.shape[1], fp(y))
    return y


def l2_norm_groups(x, h, n):
    x = f32c(x)
    y = np.empty_like(x)
    lib().orc_l2_norm_groups(fp(x), h, n, fp(y))
    return y


def dplr_update(s, k, v, w, a, b, h, n):
    s = f32c(s).copy()
    args = [f32c(t) for t in (k, v, w, a, b)]
    lib().orc_dplr_update(fp(s), *[fp(t) for t in args], h, n)
    return s


def dplr_matvec(s, r, h, n):
    s, r = f32c(s), f32c(r)
    y = np.empty(h * n, np.float32)
    lib().orc_dplr_matvec(fp(s), fp(r), h, n, fp(y))
    return y


def sum_rk_rk(r, k, rk, v, h, n):
    r, k, rk, v = f32c(r), f32c(k), f32c(rk), f32c(v)
    y = np.empty(h * n, np.float32)
    lib().orc_sum_rk_rk(fp(r), fp(k), fp(rk), fp(v), h, n, fp(y))
    return y


def argmax(x):
    x = f32c(x)
    return int(lib().orc_argmax(fp(x), x.size))


def u01(s):
    return float(lib().orc_u01(s & 0xFFFFFFFF))


def sample(logits, temperature=1.0, top_k=0, top_p=1.0, seed=0, rep=1.0, freq=0.0, pres=0.0, hist=()):
    x = f32c(logits)
    h = np.ascontiguousarray(np.asarray(hist, dtype=np.uint32)) if len(hist) else np.zeros(1, np.uint32)
    work = np.empty(2 * x.size, np.float32)
    return int(lib().orc_sample(fp(x), x.size, temperature, top_k, top_p, seed & 0xFFFFFFFF, rep, freq, pres,
                                up(h), len(hist), fp(work)))


# ------------------------------------------------------------ model
class _OrcModel(ctypes.Structure):
    _fields_ = [("n_layer", ctypes.c_int64), ("c", ctypes.c_int64), ("vocab", ctypes.c_int64),
                ("head_size", ctypes.c_int64), ("n_head", ctypes.c_int64), ("ffn", ctypes.c_int64),
                ("wm", ctypes.c_int64), ("am", ctypes.c_int64), ("vm", ctypes.c_int64), ("gm", ctypes.c_int64),
                ("emb_ln", ctypes.POINTER(ctypes.c_float)), ("ln_out_w", ctypes.POINTER(ctypes.c_float)),
                ("ln_out_b", ctypes.POINTER(ctypes.c_float)), ("head", ctypes.POINTER(ctypes.c_float)),
                ("layer", ctypes.POINTER(ctypes.POINTER(ctypes.c_float)))]


class Model:
    """Model::from_safetensors + forward (model.rs:276-517)."""

    def __init__(self, path=None, tensors=None):
        if tensors is None:
            from safetensors.numpy import load_file
            tensors = load_file(path)
        st = tensors
        names = list(st.keys())
        self.n_layer = 1 + max(int(k.split(".")[1]) for k in names if k.startswith("blocks."))
        emb = st["emb.weight"]
        self.vocab, self.c = emb.shape
        self.n_head, self.head_size = st["blocks.0.att.r_k"].shape
        c = self.c

        def mid_of(k):
            s = st[k].shape
            return s[1] if s[0] == c else s[0]

        self.wm, self.am = mid_of("blocks.0.att.w1"), mid_of("blocks.0.att.a1")
        self.vm, self.gm = mid_of("blocks.0.att.v1"), mid_of("blocks.0.att.g1")
        fk = st.get("blocks.0.ffn.key.weight")
        self.ffn = fk.shape[0] if fk is not None else st["blocks.0.ffn.key.weight.int8_idx"].shape[0]
        keep = []

        def keepa(a):
            a = f32c(a)
            keep.append(a)
            return a

        def lin(key, m, k):  # model.rs:256-273 then transpose to [in, out]
            if key in st:
                raw = st[key].astype(np.float32).reshape(m, k)
            else:
                raw = dequant_int8(st[key + ".int8_idx"], st[key + ".int8_sz"], m, k)
            return keepa(raw.T)

        def lora(key, i, o):  # model.rs:564-581
            a = st[key].astype(np.float32)
            if a.shape == (i, o):
                return keepa(a)
            if a.shape == (o, i):
                return keepa(a.T)
            raise ValueError(f"{key}: unexpected shape {a.shape}")

        embf = f32c(emb.astype(np.float32))
        ln0w = f32c(st["blocks.0.ln0.weight"].astype(np.float32).reshape(-1))
        ln0b = f32c(st["blocks.0.ln0.bias"].astype(np.float32).reshape(-1))
        self.emb_ln = np.empty_like(embf)
        lib().orc_layer_norm_rows(fp(embf), fp(ln0w), fp(ln0b), c, self.vocab, 1e-5, fp(self.emb_ln))
        del embf
        self.ln_out_w = keepa(st["ln_out.weight"].astype(np.float32).reshape(-1))
        self.ln_out_b = keepa(st["ln_out.bias"].astype(np.float32).reshape(-1))
        self.head = lin("head.weight", self.vocab, c)
        ptrs = []
        for i in range(self.n_layer):
            p = f"blocks.{i}."
            for f in FIELDS:
                key = p + f
                if f.endswith((".receptance.weight", ".key.weight", ".value.weight", ".output.weight")) and f.startswith("att."):
                    arr = lin(key, c, c)
                elif f == "ffn.key.weight":
                    arr = lin(key, self.ffn, c)
                elif f == "ffn.value.weight":
                    arr = lin(key, c, self.ffn)
                elif f in ("att.w1", "att.a1", "att.v1", "att.g1"):
                    mid = {"w": self.wm, "a": self.am, "v": self.vm, "g": self.gm}[f[4]]
                    arr = lora(key, c, mid)
                elif f in ("att.w2", "att.a2", "att.v2", "att.g2"):
                    mid = {"w": self.wm, "a": self.am, "v": self.vm, "g": self.gm}[f[4]]
                    arr = lora(key, mid, c)
                else:
                    arr = keepa(st[key].astype(np.float32).reshape(-1))
                ptrs.append(fp(arr))
        self._keep = keep
        self._ptrs = (ctypes.POINTER(ctypes.c_float) * len(ptrs))(*ptrs)
        self._m = _OrcModel(self.n_layer, c, self.vocab, self.head_size, self.n_head, self.ffn, self.wm, self.am,
                            self.vm, self.gm, fp(self.emb_ln), fp(self.ln_out_w), fp(self.ln_out_b), fp(self.head),
                            self._ptrs)

    @property
    def state_len(self):
        return self.n_layer * (2 * self.c + self.n_head * self.head_size ** 2) + self.c

    def init_state(self):
        return np.zeros(self.state_len, np.float32)

    def forward(self, tokens, state):
        """Advances `state` in place over tokens; returns the last logits."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        logits = np.empty(self.vocab, np.float32)
        lib().orc_forward(ctypes.byref(self._m), up(t), t.size, fp(state), fp(logits))
        return logits

    def greedy(self, prompt, n, state=None):
        """Prompt then n greedy tokens; returns (tokens, per-step logits list, state)."""
        st = self.init_state() if state is None else state
        lg = self.forward(prompt, st)
        toks, lgs = [], [lg]
        for _ in range(n):
            t = argmax(lg)
            toks.append(t)
            lg = self.forward([t], st)
            lgs.append(lg)
        return toks, lgs, st
