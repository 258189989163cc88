"""Seeded synthetic RWKV-7 models in the reference's safetensors layout.

Key names, shapes and dtypes follow what the reference loads
(model.rs:276-346, 534-620; gpu_model.rs:401-546, 3260-3568):

    emb.weight [V, C]; blocks.0.ln0.{weight,bias} [C]; ln_out.{weight,bias} [C]
    head.weight [V, C]  (or head.weight.int8_idx U8 [V, C] + .int8_sz U32 [V, C/128])
    blocks.i.ln1/ln2.{weight,bias} [C]; att.ln_x.{weight,bias} [C]
    blocks.i.att.{x_r,x_w,x_k,x_v,x_a,x_g,w0,a0,v0,k_k,k_a} [1, 1, C]; att.r_k [H, N]
    blocks.i.att.{w1,a1,v1,g1} [C, mid]; att.{w2,a2,v2,g2} [mid, C]
    blocks.i.att.{receptance,key,value,output}.weight [C, C]   ([out, in])
    blocks.i.ffn.x_k [1, 1, C]; ffn.key.weight [F, C]; ffn.value.weight [C, F]

Random init (the benchmark configs' recipe): every tensor N(0, 0.02^2) drawn
from numpy's PCG64 seeded with `seed`, tensors visited in `key_order()`;
LayerNorm / GroupNorm weights are 1 and biases 0.

int8 layout (model.rs:230-252): idx[m, k] u8, sz[m, k/128] u32 with the fp16
scale in the low 16 bits and the fp16 zero in the high 16 bits.  `quantize_rows`
produces the symmetric per-output-row absmax variant as reference-format
groups: q_u8 = q_s8 + 128, scale = f16(absmax/127), zero = -128*scale (exact
in fp16), repeated for every 128-group of the row, so the stored weight is
exactly scale * q_s8.
"""
import json
import os
import struct

import numpy as np

TINY = dict(n_layer=12, c=768, vocab=65536, n_head=12, head_size=64, ffn=3072, wm=64, am=64, vm=32, gm=128)
THREE_B = dict(n_layer=32, c=2560, vocab=65536, n_head=40, head_size=64, ffn=10240, wm=96, am=96, vm=64, gm=256)

LINEARS = ("att.receptance.weight", "att.key.weight", "att.value.weight", "att.output.weight",
           "ffn.key.weight", "ffn.value.weight")


def shapes(cfg):
    """(key, shape) pairs in the fixed generation order."""
    c, v, h, n, f = cfg["c"], cfg["vocab"], cfg["n_head"], cfg["head_size"], cfg["ffn"]
    out = [("emb.weight", (v, c)), ("blocks.0.ln0.weight", (c,)), ("blocks.0.ln0.bias", (c,))]
    for i in range(cfg["n_layer"]):
        p = f"blocks.{i}."
        out += [(p + "ln1.weight", (c,)), (p + "ln1.bias", (c,)), (p + "ln2.weight", (c,)), (p + "ln2.bias", (c,))]
        for nm in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g", "w0", "a0", "v0", "k_k", "k_a"):
            out.append((p + "att." + nm, (1, 1, c)))
        out.append((p + "att.r_k", (h, n)))
        for nm, mid in (("w", cfg["wm"]), ("a", cfg["am"]), ("v", cfg["vm"]), ("g", cfg["gm"])):
            out += [(p + f"att.{nm}1", (c, mid)), (p + f"att.{nm}2", (mid, c))]
        out += [(p + "att.receptance.weight", (c, c)), (p + "att.key.weight", (c, c)),
                (p + "att.value.weight", (c, c)), (p + "att.output.weight", (c, c)),
                (p + "att.ln_x.weight", (c,)), (p + "att.ln_x.bias", (c,)),
                (p + "ffn.x_k", (1, 1, c)), (p + "ffn.key.weight", (f, c)), (p + "ffn.value.weight", (c, f))]
    out += [("ln_out.weight", (c,)), ("ln_out.bias", (c,)), ("head.weight", (v, c))]
    return out


def key_order(cfg):
    return [k for k, _ in shapes(cfg)]


def _is_norm(key):
    return key.endswith(("ln0.weight", "ln0.bias", "ln1.weight", "ln1.bias", "ln2.weight", "ln2.bias",
                         "ln_x.weight", "ln_x.bias", "ln_out.weight", "ln_out.bias"))


def _f16_bits(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16).astype(np.uint32)


def quantize_rows(w):
    """Symmetric per-row absmax int8 in the reference group format.
    Returns (idx u8 [m,k], sz u32 [m,k/128])."""
    w = np.asarray(w, dtype=np.float32)
    m, k = w.shape
    assert k % 128 == 0, "int8 rows need k % 128 == 0"
    amax = np.abs(w).max(axis=1)
    s16 = (amax / np.float32(127.0)).astype(np.float16)
    s16 = np.where(s16 == 0, np.float16(1.0), s16)
    s32 = s16.astype(np.float32)
    q = np.clip(np.rint(w / s32[:, None]), -127, 127).astype(np.int16)
    idx = (q + 128).astype(np.uint8)
    zero = (-128.0 * s32).astype(np.float16)
    assert np.all(zero.astype(np.float32) == -128.0 * s32), "zero must be exact in fp16"
    word = (zero.view(np.uint16).astype(np.uint32) << 16) | s16.view(np.uint16).astype(np.uint32)
    sz = np.repeat(word[:, None], k // 128, axis=1)
    return idx, np.ascontiguousarray(sz)


def quantize_groups(w):
    """Asymmetric per-group-128 min/max int8 (the reference quantiser's scheme,
    model.rs:886-912 / tools/quantize_any4.py:241-301)."""
    w = np.asarray(w, dtype=np.float32)
    m, k = w.shape
    g = w.reshape(m, k // 128, 128)
    mn = g.min(axis=2)
    mx = g.max(axis=2)
    sc = ((mx - mn) / np.float32(255.0)).astype(np.float32)
    s16 = sc.astype(np.float16)
    z16 = mn.astype(np.float16)
    inv = np.where(sc <= 0, np.float32(1.0), np.float32(1.0) / np.where(sc <= 0, 1, sc))
    q = np.clip(np.rint((g - mn[..., None]) * inv[..., None]), 0, 255).astype(np.uint8).reshape(m, k)
    sz = (z16.view(np.uint16).astype(np.uint32) << 16) | s16.view(np.uint16).astype(np.uint32)
    return q, np.ascontiguousarray(sz)


def dequant(idx, sz):
    """fp32 dequant w = scale*q + zero (numpy mirror of model.rs:234-252)."""
    m, k = idx.shape
    s = sz.astype(np.uint32)
    scale = (s & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32)
    zero = (s >> 16).astype(np.uint16).view(np.float16).astype(np.float32)
    q = idx.astype(np.float32).reshape(m, k // 128, 128)
    return (scale[..., None] * q + zero[..., None]).reshape(m, k).astype(np.float32)


class _Writer:
    """Streams tensors into a safetensors file (header first, then data)."""

    def __init__(self, path, entries):
        # entries: list of (key, dtype str, shape, nbytes)
        header = {}
        off = 0
        for key, dt, shape, nbytes in entries:
            header[key] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + nbytes]}
            off += nbytes
        hb = json.dumps(header, separators=(",", ":")).encode()
        hb += b" " * ((8 - len(hb) % 8) % 8)
        self.f = open(path, "wb")
        self.f.write(struct.pack("<Q", len(hb)))
        self.f.write(hb)

    def write(self, arr):
        self.f.write(np.ascontiguousarray(arr).tobytes())

    def close(self):
        self.f.close()


def write_model(path, cfg, seed=0, linear="f32", head="f32", emb="f32", lora="f32", group_quant=False):
    """Generates and writes a model.

    linear/head: "f32", "f16" or "i8" (int8 reference format); emb/lora:
    "f32" or "f16".  group_quant=True uses asymmetric per-group quantisation
    instead of the symmetric per-row variant.
    """
    rng = np.random.Generator(np.random.PCG64(seed))
    items = shapes(cfg)
    quant = quantize_groups if group_quant else quantize_rows
    entries = []
    kinds = {}
    for key, shp in items:
        is_lin = key.endswith(LINEARS)
        fmt = "f32"
        if key == "head.weight":
            fmt = head
        elif is_lin:
            fmt = linear
        elif key == "emb.weight":
            fmt = emb
        elif any(key.endswith(f"att.{n}{d}") for n in "wavg" for d in "12"):
            fmt = lora
        kinds[key] = fmt
        n = int(np.prod(shp))
        if fmt == "i8":
            m, k = shp
            entries.append((key + ".int8_idx", "U8", (m, k), m * k))
            entries.append((key + ".int8_sz", "U32", (m, k // 128), m * k // 128 * 4))
        elif fmt == "f16":
            entries.append((key, "F16", shp, n * 2))
        else:
            entries.append((key, "F32", shp, n * 4))
    w = _Writer(path, entries)
    try:
        for key, shp in items:
            if _is_norm(key):
                arr = np.ones(shp, np.float32) if key.endswith("weight") else np.zeros(shp, np.float32)
            else:
                arr = rng.standard_normal(shp, dtype=np.float32) * np.float32(0.02)
            fmt = kinds[key]
            if fmt == "i8":
                idx, sz = quant(arr)
                w.write(idx)
                w.write(sz)
            elif fmt == "f16":
                w.write(arr.astype(np.float16))
            else:
                w.write(arr)
    finally:
        w.close()
    return path


def prompt(cfg, n, seed=0, stream=1):
    """Uniform random token ids from PCG64 seeded with (seed, stream)."""
    rng = np.random.Generator(np.random.PCG64([seed, stream]))
    return rng.integers(0, cfg["vocab"], size=n, dtype=np.int64).astype(np.uint32)
