"""MiniCPM-shaped decoder configuration and seeded synthetic weights.

The program this mirrors is the one tools/p12_build_minicpm.py:766-981 emits
(and tools/p14_gen_build.py:470-560 closes with in-engine argmax): per layer
RMSNORM -> int8 GEMM q/k/v (per-output-row f32 scale, the 4th operand of
OP_GEMM, core/src/interp.rs:765-801) -> per-head RoPE / scaled causal softmax
attention -> GEMM o -> residual -> RMSNORM -> GEMM gate/up -> SiLU * up ->
GEMM down -> residual; final RMSNORM and a bf16 LM head (OP_GEMM bf16 path,
core/src/interp.rs:752-764); token ids enter through OP_EMB over a bf16 table.

Weights are random-init with the distributions the benchmark fixes: int8
weights uniform in [-127, 127], per-row scale |N(0, 0.02)|/127 + 1e-6, norm
gains 1.0, bf16 embedding and LM head N(0, 1)*0.02 rounded to nearest even.
"""
from __future__ import annotations

import numpy as np

MINICPM_2B = dict(n_layers=40, hidden=2304, n_heads=36, head_dim=64, inter=5760,
                  vocab=122753, eps=1e-5, theta=10000.0)

LAYER_KEYS = ("wq", "wk", "wv", "wo", "wg", "wu", "wd",
              "sq", "sk", "sv", "so", "sg", "su", "sd", "in_ln", "post_ln")


def finish_config(cfg: dict) -> dict:
    cfg = dict(cfg)
    cfg.setdefault("head_dim", cfg["hidden"] // cfg["n_heads"])
    cfg.setdefault("eps", 1e-5)
    cfg.setdefault("theta", 10000.0)
    # scale1 = 1/sqrt(HD) emitted as an f32 constant (p12_build_minicpm.py:350)
    cfg["attn_scale"] = float(np.float32(1.0 / np.sqrt(cfg["head_dim"])))
    if cfg["n_heads"] * cfg["head_dim"] != cfg["hidden"]:
        raise ValueError("hidden must equal n_heads * head_dim")
    return cfg


def minicpm_2b_config() -> dict:
    return finish_config(MINICPM_2B)


def tiny_config(n_layers=2, hidden=128, n_heads=2, inter=256, vocab=500) -> dict:
    return finish_config(dict(n_layers=n_layers, hidden=hidden, n_heads=n_heads,
                              inter=inter, vocab=vocab))


def bf16_rne(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits, round to nearest even (tensor/src/dtype.rs:40-46)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    return ((u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)).astype(np.uint16)


def uniform_int8(rng: np.random.Generator, shape) -> np.ndarray:
    """Uniform integers in [-127, 127]: random bytes u in [0, 254] shifted by
    -127; the byte value 255 is redrawn (exact uniformity, ~1/256 redraws)."""
    n = int(np.prod(shape))

    def raw_bytes(count):
        return rng.bit_generator.random_raw((count + 7) // 8).view(np.uint8)[:count]

    u = raw_bytes(n)
    bad = np.flatnonzero(u == 255)
    while bad.size:
        u[bad] = raw_bytes(bad.size)
        bad = bad[u[bad] == 255]
    u -= np.uint8(127)  # wraps: 0..126 -> 129..255 (= -127..-1), 127..254 -> 0..127
    return u.view(np.int8).reshape(shape)


def q8_weight(rng: np.random.Generator, n: int, k: int):
    q = uniform_int8(rng, (n, k))
    s = (np.abs(rng.standard_normal(n, dtype=np.float32) * np.float32(0.02)) / np.float32(127)
         + np.float32(1e-6)).astype(np.float32)
    return q, s


def make_weights(cfg: dict, seed: int = 3, threads: int = 8) -> dict:
    """Seeded host weights; layer arrays are [N, K] row-major (nn.Linear).

    Every layer and every 8192-row block of the two bf16 tables draws from its
    own child of SeedSequence(seed), so the values depend only on the seed and
    the shapes, not on the thread count used to fill them."""
    from concurrent.futures import ThreadPoolExecutor
    H, I, V = cfg["hidden"], cfg["inter"], cfg["vocab"]
    nl = cfg["n_layers"]
    step = 8192
    nblk = (V + step - 1) // step
    kids = np.random.SeedSequence(seed).spawn(nl + 2 * nblk)

    def layer(li):
        rng = np.random.default_rng(kids[li])
        L = {}
        for name, (n, k) in (("q", (H, H)), ("k", (H, H)), ("v", (H, H)), ("o", (H, H)),
                             ("g", (I, H)), ("u", (I, H)), ("d", (H, I))):
            L["w" + name], L["s" + name] = q8_weight(rng, n, k)
        L["in_ln"] = np.ones(H, np.float32)
        L["post_ln"] = np.ones(H, np.float32)
        return L

    embed = np.empty((V, H), np.uint16)
    lm_head = np.empty((V, H), np.uint16)

    def table_block(t, b):
        rng = np.random.default_rng(kids[nl + t * nblk + b])
        r0 = b * step
        rows = min(step, V - r0)
        blk = rng.standard_normal((rows, H), dtype=np.float32) * np.float32(0.02)
        (embed if t == 0 else lm_head)[r0:r0 + rows] = bf16_rne(blk)

    with ThreadPoolExecutor(max(1, threads)) as ex:
        layers = list(ex.map(layer, range(nl)))
        list(ex.map(lambda tb: table_block(*tb), [(t, b) for t in (0, 1) for b in range(nblk)]))
    return dict(layers=layers, embed=embed, lm_head=lm_head,
                final_norm=np.ones(H, np.float32))


def make_prompts(cfg: dict, batch: int, S: int, seed: int = 3) -> np.ndarray:
    rng = np.random.default_rng(seed + 1000)
    return rng.integers(0, cfg["vocab"], size=(batch, S), dtype=np.int32)
