"""Seeded synthetic OLMo-3-shaped models for the parity tests.

Weights are drawn with numpy's PCG64 from fixed seeds (N(0, 0.02) for the
projections and the embedding, U(0.5, 1.5) for the norm and QK-norm weights,
as BASELINE.json's configs ask), stored in the requested format, and handed
both to the oracle (as views) and to the HIP engine (as uploads).

`ref64_forward` is an independent float64 numpy transformer used to pin the
oracle's model wiring (post-norm order, residuals, QK-norm, YaRN RoPE, GQA
head mapping, sliding window); it shares no code with oracle/oracle.c.
"""
from __future__ import annotations

import numpy as np

LIN_NAMES = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")


def tiny_config(**kw) -> dict:
    cfg = dict(vocab=256, d_model=64, n_layers=2, n_heads=4, n_kv_heads=2,
               ffn_hidden=128, max_seq=128, rope_theta=10000.0, rms_eps=1e-5,
               yarn=None, sliding_window=0, layer_sliding=None, post_norm=True,
               qk_norm=True)
    cfg.update(kw)
    return cfg


def olmo3_small_config(**kw) -> dict:
    """OLMo-3 wiring (post-norm, QK-norm, YaRN, SWA on layers i % 4 != 3) at a
    size the oracle finishes in well under a second per token."""
    cfg = dict(vocab=512, d_model=256, n_layers=4, n_heads=4, n_kv_heads=4,
               ffn_hidden=512, max_seq=256, rope_theta=500000.0, rms_eps=1e-6,
               yarn=dict(factor=8.0, orig_max_pos=8192, attn_factor=1.2079441541679836,
                         beta_fast=32.0, beta_slow=1.0),
               sliding_window=16, layer_sliding=None, post_norm=True, qk_norm=True)
    cfg.update(kw)
    if cfg["layer_sliding"] is None:
        cfg["layer_sliding"] = [0 if i % 4 == 3 else 1 for i in range(cfg["n_layers"])]
    return cfg


def shapes(cfg):
    d, hd = cfg["d_model"], cfg["d_model"] // cfg["n_heads"]
    kv = cfg["n_kv_heads"] * hd
    f = cfg["ffn_hidden"]
    return dict(wq=(d, d), wk=(kv, d), wv=(kv, d), wo=(d, d),
                w_gate=(f, d), w_up=(f, d), w_down=(d, f)), hd


def make_weights(cfg: dict, seed: int = 1234, fmt: str = "bf16", block: int = 32) -> dict:
    """Returns {'f32': dequantised weights (what the reference computes with),
    'stored': the stored form per matrix (fmt, arrays), 'norms': ...}."""
    import oracle as orc
    rng = np.random.default_rng(seed)
    shp, hd = shapes(cfg)
    d, V, L = cfg["d_model"], cfg["vocab"], cfg["n_layers"]

    def store(w):
        if fmt == "f32":
            return ("f32", (w,)), w
        if fmt == "bf16":
            bits = orc.bf16_from_f32(w)
            return ("bf16", (bits,)), orc.bf16_to_f32(bits)
        if fmt == "int8":
            q, s = orc.int8_quantize(w)
            return ("int8", (q, s)), orc.int8_dequantize(q, s)
        if fmt == "int4":
            q, s = orc.int4_quantize(w, block)
            return ("int4", (q, s)), orc.int4_dequantize(q, s, w.shape[0], w.shape[1], block)
        raise ValueError(fmt)

    out = dict(cfg=cfg, fmt=fmt, block=block, layers=[])
    emb = (rng.standard_normal((V, d)) * 0.02).astype(np.float32)
    bits = orc.bf16_from_f32(emb)
    out["embed_bits"] = bits                       # embedding kept as bf16
    out["embed"] = orc.bf16_to_f32(bits)
    lm = (rng.standard_normal((V, d)) * 0.02).astype(np.float32)
    out["lm_head_stored"], out["lm_head"] = store(lm)
    out["final_norm"] = rng.uniform(0.5, 1.5, d).astype(np.float32)
    for _ in range(L):
        lw = {}
        for n in LIN_NAMES:
            w = (rng.standard_normal(shp[n]) * 0.02).astype(np.float32)
            lw[n + "_stored"], lw[n] = store(w)
        lw["attn_norm"] = rng.uniform(0.5, 1.5, d).astype(np.float32)
        lw["ffn_norm"] = rng.uniform(0.5, 1.5, d).astype(np.float32)
        if cfg.get("qk_norm", True):
            lw["q_norm"] = rng.uniform(0.5, 1.5, cfg["n_heads"] * hd).astype(np.float32)
            lw["k_norm"] = rng.uniform(0.5, 1.5, cfg["n_kv_heads"] * hd).astype(np.float32)
        else:
            lw["q_norm"] = lw["k_norm"] = None
        out["layers"].append(lw)
    return out


def _view(stored, rows, cols, block):
    import oracle as orc
    kind, arrs = stored
    if kind == "f32":
        return orc.MatView.f32(arrs[0])
    if kind == "bf16":
        return orc.MatView.bf16(arrs[0], rows, cols)
    if kind == "int8":
        return orc.MatView.int8(arrs[0], arrs[1])
    return orc.MatView.int4(arrs[0], arrs[1], rows, cols, block)


def oracle_model(W: dict, threads: int = 1, slots: int = 1):
    import oracle as orc
    cfg = W["cfg"]
    shp, _ = shapes(cfg)
    V, d = cfg["vocab"], cfg["d_model"]
    layers = []
    for lw in W["layers"]:
        ld = {n: _view(lw[n + "_stored"], *shp[n], W["block"]) for n in LIN_NAMES}
        ld.update(attn_norm=lw["attn_norm"], ffn_norm=lw["ffn_norm"],
                  q_norm=lw["q_norm"], k_norm=lw["k_norm"])
        layers.append(ld)
    weights = dict(embed=orc.MatView.bf16(W["embed_bits"], V, d),
                   lm_head=_view(W["lm_head_stored"], V, d, W["block"]),
                   final_norm=W["final_norm"], layers=layers)
    return orc.Model(cfg, weights, threads=threads, slots=slots)


# ---------------------------------------------------------------------------
# independent float64 reference (pins the oracle's model wiring)
# ---------------------------------------------------------------------------

class Ref64:
    def __init__(self, W: dict):
        self.W, self.cfg = W, W["cfg"]
        c = self.cfg
        self.hd = c["d_model"] // c["n_heads"]
        half = self.hd // 2
        i = np.arange(half, dtype=np.float64)
        base = 1.0 / c["rope_theta"] ** (2.0 * i / self.hd)
        f = base.copy()
        y = c.get("yarn")
        if y:
            wl = 2 * np.pi / base
            low = y["orig_max_pos"] / (2 * np.pi * y["beta_slow"])
            high = y["orig_max_pos"] / (2 * np.pi * y["beta_fast"])
            for j in range(half):
                if wl[j] < high:
                    f[j] = base[j]
                elif wl[j] > low:
                    f[j] = base[j] / y["factor"]
                else:
                    a = (wl[j] - high) / (low - high)
                    f[j] = base[j] / (a * y["factor"] + 1 - a)
        self.freqs = f
        self.scale = (y["attn_factor"] if y else 1.0) / np.sqrt(self.hd)
        L, kvd = c["n_layers"], c["n_kv_heads"] * self.hd
        self.K = np.zeros((L, c["max_seq"], kvd))
        self.Vc = np.zeros((L, c["max_seq"], kvd))
        self.pos = 0

    @staticmethod
    def _rms(x, w, eps):
        return x / np.sqrt(np.mean(x * x) + eps) * w

    def _rope(self, x, pos):
        h = self.hd // 2
        a = pos * self.freqs
        c, s = np.cos(a), np.sin(a)
        x0, x1 = x[..., :h].copy(), x[..., h:].copy()
        return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)

    def forward_one(self, tok):
        c, W = self.cfg, self.W
        pos = self.pos
        self.pos += 1
        H, KVH, hd, d = c["n_heads"], c["n_kv_heads"], self.hd, c["d_model"]
        x = W["embed"][min(tok, c["vocab"] - 1)].astype(np.float64)
        sl = c.get("layer_sliding") or [0] * c["n_layers"]
        for li, lw in enumerate(W["layers"]):
            g = lambda n: lw[n].astype(np.float64)  # noqa: E731

            def attn(xin):
                q = (g("wq") @ xin).reshape(H, hd)
                k = (g("wk") @ xin).reshape(KVH, hd)
                v = (g("wv") @ xin).reshape(KVH, hd)
                if lw["q_norm"] is not None:
                    qn = lw["q_norm"].astype(np.float64).reshape(H, hd)
                    kn = lw["k_norm"].astype(np.float64).reshape(KVH, hd)
                    q = q / np.sqrt(np.mean(q * q, axis=1, keepdims=True) + 1e-6) * qn
                    k = k / np.sqrt(np.mean(k * k, axis=1, keepdims=True) + 1e-6) * kn
                q, k = self._rope(q, pos), self._rope(k, pos)
                self.K[li, pos] = k.reshape(-1)
                self.Vc[li, pos] = v.reshape(-1)
                Kc = self.K[li, :pos + 1].reshape(pos + 1, KVH, hd)
                Vc = self.Vc[li, :pos + 1].reshape(pos + 1, KVH, hd)
                w = c.get("sliding_window") or 0
                lo = pos - w + 1 if (sl[li] and w > 0 and pos - w + 1 > 0) else 0
                out = np.zeros((H, hd))
                for h in range(H):
                    kvh = h // (H // KVH)
                    s = Kc[lo:, kvh] @ q[h] * self.scale
                    p = np.exp(s - s.max())
                    p /= p.sum()
                    out[h] = p @ Vc[lo:, kvh]
                return g("wo") @ out.reshape(-1)

            def ffn(xin):
                gt, up = g("w_gate") @ xin, g("w_up") @ xin
                return g("w_down") @ (gt / (1 + np.exp(-gt)) * up)

            an, fn = lw["attn_norm"].astype(np.float64), lw["ffn_norm"].astype(np.float64)
            if c.get("post_norm", True):
                x = x + self._rms(attn(x), an, c["rms_eps"])
                x = x + self._rms(ffn(x), fn, c["rms_eps"])
            else:
                x = x + attn(self._rms(x, an, c["rms_eps"]))
                x = x + ffn(self._rms(x, fn, c["rms_eps"]))
        x = self._rms(x, W["final_norm"].astype(np.float64), c["rms_eps"])
        return W["lm_head"].astype(np.float64) @ x


# ---------------------------------------------------------------------------
# the same weights uploaded into the HIP engine
# ---------------------------------------------------------------------------

def engine_model(W: dict, max_batch: int = 1, use_graph: bool = True):
    from atlas_amd import model as am
    c = W["cfg"]
    y = c.get("yarn")
    sl = c.get("layer_sliding") or [0] * c["n_layers"]
    cfg = am.ModelConfig(vocab_size=c["vocab"], d_model=c["d_model"], n_layers=c["n_layers"],
                         n_heads=c["n_heads"], n_kv_heads=c["n_kv_heads"],
                         ffn_hidden=c["ffn_hidden"], max_seq_len=c["max_seq"],
                         rope_theta=c["rope_theta"], rms_norm_eps=c["rms_eps"],
                         layer_types=["sliding" if s else "full" for s in sl],
                         sliding_window=c.get("sliding_window") or None,
                         rope_scaling=am.RopeYarn(**y) if y else None,
                         post_norm=c.get("post_norm", True), qk_norm=c.get("qk_norm", True))
    fmt = {"bf16": am.W_BF16, "int8": am.W_INT8, "int4": am.W_INT4}[W["fmt"]]
    m = am.OlmoModel(cfg, weight_format=fmt, int4_block=W["block"], max_batch=max_batch)
    m.use_graph(use_graph)
    kinds = dict(wq=am.T_WQ, wk=am.T_WK, wv=am.T_WV, wo=am.T_WO, w_gate=am.T_W_GATE,
                 w_up=am.T_W_UP, w_down=am.T_W_DOWN)

    def put(kind, layer, stored):
        k, arrs = stored
        m.set_tensor(kind, layer, arrs[0], arrs[1] if len(arrs) > 1 else None)

    for li, lw in enumerate(W["layers"]):
        for n, kd in kinds.items():
            put(kd, li, lw[n + "_stored"])
        m.set_tensor(am.T_ATTN_NORM, li, lw["attn_norm"])
        m.set_tensor(am.T_FFN_NORM, li, lw["ffn_norm"])
        if lw["q_norm"] is not None:
            m.set_tensor(am.T_Q_NORM, li, lw["q_norm"])
            m.set_tensor(am.T_K_NORM, li, lw["k_norm"])
    m.set_tensor(am.T_EMBED, 0, W["embed_bits"])
    put(am.T_LM_HEAD, 0, W["lm_head_stored"])
    m.set_tensor(am.T_FINAL_NORM, 0, W["final_norm"])
    return m
