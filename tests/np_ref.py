"""Independent float64 numpy statement of the RWKV-7 step (test-only).

Written from the model's mathematics, vectorised per head, sharing no code
with oracle/rsv_oracle.c: it pins the oracle's whole-model forward against a
dropped term, a transposed operand or a wrong index.
"""
import numpy as np


def _f64(a):
    return np.asarray(a, dtype=np.float64)


def _ln(x, w, b, eps):
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def _dequant(idx, sz):
    m, k = idx.shape
    s = sz.astype(np.uint32)
    sc = (s & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
    ze = (s >> 16).astype(np.uint16).view(np.float16).astype(np.float64)
    q = idx.astype(np.float64).reshape(m, k // 128, 128)
    return (sc[..., None] * q + ze[..., None]).reshape(m, k)


class NpModel:
    def __init__(self, st):
        def W(key):  # [out, in] float64
            if key in st:
                return _f64(st[key])
            return _dequant(st[key + ".int8_idx"], st[key + ".int8_sz"])

        self.emb = _f64(st["emb.weight"])
        self.V, self.C = self.emb.shape
        self.H, self.N = st["blocks.0.att.r_k"].shape
        self.L = 1 + max(int(k.split(".")[1]) for k in st if k.startswith("blocks."))
        self.emb_ln = _ln(self.emb, _f64(st["blocks.0.ln0.weight"]), _f64(st["blocks.0.ln0.bias"]), 1e-5)
        self.head = W("head.weight")
        self.lo_w, self.lo_b = _f64(st["ln_out.weight"]), _f64(st["ln_out.bias"])
        self.layers = []
        for i in range(self.L):
            p = f"blocks.{i}."
            g = lambda k: _f64(st[p + k]).reshape(-1)
            lay = {k: g(k) for k in ["ln1.weight", "ln1.bias", "ln2.weight", "ln2.bias", "att.x_r", "att.x_w",
                                     "att.x_k", "att.x_v", "att.x_a", "att.x_g", "att.w0", "att.a0", "att.v0",
                                     "att.r_k", "att.k_k", "att.k_a", "att.ln_x.weight", "att.ln_x.bias", "ffn.x_k"]}
            for nm in "wavg":
                a1, a2 = _f64(st[p + f"att.{nm}1"]), _f64(st[p + f"att.{nm}2"])
                lay[nm + "1"] = a1 if a1.shape[0] == self.C else a1.T  # [C, mid]
                lay[nm + "2"] = a2 if a2.shape[1] == self.C else a2.T  # [mid, C]
            for nm in ["att.receptance.weight", "att.key.weight", "att.value.weight", "att.output.weight",
                       "ffn.key.weight", "ffn.value.weight"]:
                lay[nm] = W(p + nm)
            self.layers.append(lay)

    def state(self):
        return [dict(tx=np.zeros(self.C), S=np.zeros((self.H, self.N, self.N)), cx=np.zeros(self.C))
                for _ in range(self.L)]

    def step(self, tok, st):
        H, N = self.H, self.N
        x = self.emb_ln[tok].copy()
        vfirst = None
        for i, L in enumerate(self.layers):
            s = st[i]
            xn = _ln(x, L["ln1.weight"], L["ln1.bias"], 1e-5)
            d = s["tx"] - xn
            s["tx"] = xn
            mix = {c: xn + d * L["att.x_" + c] for c in "rwkvag"}
            r = L["att.receptance.weight"] @ mix["r"]
            k = L["att.key.weight"] @ mix["k"]
            v = L["att.value.weight"] @ mix["v"]
            if vfirst is None:
                vfirst = v
            else:
                gate = 1 / (1 + np.exp(-(L["att.v0"] + (mix["v"] @ L["v1"]) @ L["v2"])))
                v = v * (1 - gate) + vfirst * gate
            w = np.exp(-np.exp(-0.5) / (1 + np.exp(-(L["att.w0"] + np.tanh(mix["w"] @ L["w1"]) @ L["w2"]))))
            a = 1 / (1 + np.exp(-(L["att.a0"] + (mix["a"] @ L["a1"]) @ L["a2"])))
            g = (1 / (1 + np.exp(-(mix["g"] @ L["g1"])))) @ L["g2"]
            kk = (k * L["att.k_k"]).reshape(H, N)
            kk = kk / np.maximum(np.linalg.norm(kk, axis=1, keepdims=True), 1e-12)
            kmod = k * (1 + (a - 1) * L["att.k_a"])
            rh, kh, vh, wh, ah = (t.reshape(H, N) for t in (r, kmod, v, w, a))
            S = s["S"]
            # S <- S diag(w) + (S kk)(-kk*a)^T + v k^T
            S = S * wh[:, None, :] + np.einsum("hij,hj->hi", S, kk)[:, :, None] * (-kk * ah)[:, None, :] \
                + vh[:, :, None] * kh[:, None, :]
            s["S"] = S
            y = np.einsum("hij,hj->hi", S, rh)
            y = _ln(y, L["att.ln_x.weight"].reshape(H, N), L["att.ln_x.bias"].reshape(H, N), 64e-5)
            y = y + (rh * kh * L["att.r_k"].reshape(H, N)).sum(axis=1, keepdims=True) * vh
            x = x + L["att.output.weight"] @ (y.reshape(-1) * g)
            xn = _ln(x, L["ln2.weight"], L["ln2.bias"], 1e-5)
            xb = xn + (s["cx"] - xn) * L["ffn.x_k"]
            s["cx"] = xn
            x = x + L["ffn.value.weight"] @ (np.maximum(L["ffn.key.weight"] @ xb, 0) ** 2)
        return self.head @ _ln(x, self.lo_w, self.lo_b, 1e-5), vfirst

    def flat_state(self, st, vfirst):
        parts = []
        for s in st:
            parts += [s["tx"], s["S"].reshape(-1), s["cx"]]
        parts.append(vfirst)
        return np.concatenate(parts)
