"""MiniCPM-shaped decoder session on the MI355X (layer 3 of include/vmlm_hip.h).

Runs the program tools/p12_build_minicpm.py emits, closed by the in-engine
greedy loop of tools/p14_gen_build.py: prefill S prompt tokens per
sequence, take the argmax of the last row (t0), then decode steps that feed
each argmax back (t1, t2, ...). Weights, KV cache, position and tokens stay
in HBM; each decode step is one HIP graph replay.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _abi, check, lib


class Decoder:
    def __init__(self, cfg: dict, batch: int = 1, cap: int = 1024):
        self.cfg = dict(cfg)
        self.batch = int(batch)
        self.cap = int(cap)
        c = _abi.DecoderCfg(cfg["n_layers"], cfg["hidden"], cfg["n_heads"], cfg["head_dim"],
                            cfg["inter"], cfg["vocab"], self.batch, self.cap, cfg["eps"],
                            cfg["theta"], cfg["attn_scale"])
        h = C.c_void_p()
        check(lib().vmlm_decoder_create(C.byref(c), C.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            lib().vmlm_decoder_destroy(self._h)
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

    # ------------------------------------------------------------ weights
    def load(self, weights: dict) -> None:
        L = lib()
        for li, Lw in enumerate(weights["layers"]):
            a = [np.ascontiguousarray(Lw[k]) for k in
                 ("wq", "sq", "wk", "sk", "wv", "sv", "wo", "so", "wg", "sg", "wu", "su",
                  "wd", "sd", "in_ln", "post_ln")]
            check(L.vmlm_decoder_load_layer(self._h, li, *[x.ctypes.data for x in a]))
        e = np.ascontiguousarray(weights["embed"], np.uint16)
        m = np.ascontiguousarray(weights["lm_head"], np.uint16)
        f = np.ascontiguousarray(weights["final_norm"], np.float32)
        check(L.vmlm_decoder_load_globals(self._h, e.ctypes.data, m.ctypes.data, f.ctypes.data))

    # ------------------------------------------------------------ running
    def set_fused(self, enable: bool) -> None:
        """Fused five-launch layers (default at batch <= 5) or the k-slice
        eight-launch program."""
        check(lib().vmlm_decoder_set_fused(self._h, int(bool(enable))))

    @property
    def fused(self) -> bool:
        return bool(lib().vmlm_decoder_fused(self._h))

    KSLICE, FUSED, FULLK = 0, 1, 2

    def set_program(self, program: int) -> None:
        """The layer program: KSLICE (k-slice GEMVs, eight launches per
        layer), FUSED (batch <= 5, five launches) or FULLK (batch <= 16, full-K
        q/k/v and gate/up, seven launches)."""
        check(lib().vmlm_decoder_set_program(self._h, int(program)))

    @property
    def program(self) -> int:
        return int(lib().vmlm_decoder_program(self._h))

    def set_graph(self, enable: bool) -> None:
        check(lib().vmlm_decoder_set_graph(self._h, int(bool(enable))))

    def prefill(self, tokens: np.ndarray, want_logits: bool = False):
        """tokens [batch, S] int32 -> (t0 [batch], logits [batch, vocab] | None)."""
        t = np.ascontiguousarray(tokens, np.int32).reshape(self.batch, -1)
        first = np.empty(self.batch, np.int32)
        logits = np.empty((self.batch, self.cfg["vocab"]), np.float32) if want_logits else None
        check(lib().vmlm_decoder_prefill(self._h, t.ctypes.data, t.shape[1], first.ctypes.data,
                                         logits.ctypes.data if want_logits else None))
        return first, logits

    def decode(self, n_steps: int, want_tokens: bool = True, want_logits: bool = False):
        """n greedy steps -> (tokens [n, batch] | None, logits [batch, vocab] | None)."""
        toks = np.empty((n_steps, self.batch), np.int32) if want_tokens else None
        logits = np.empty((self.batch, self.cfg["vocab"]), np.float32) if want_logits else None
        check(lib().vmlm_decoder_decode(self._h, int(n_steps),
                                        toks.ctypes.data if want_tokens else None,
                                        logits.ctypes.data if want_logits else None))
        return toks, logits

    def generate(self, prompts: np.ndarray, n_steps: int):
        """Greedy chain per sequence: [t0, t1, ..., t_n] as [batch, n+1]."""
        t0, _ = self.prefill(prompts)
        toks, _ = self.decode(n_steps)
        return np.concatenate([t0[None, :], toks], 0).T.copy()

    def position(self) -> int:
        p = C.c_uint32()
        check(lib().vmlm_decoder_position(self._h, C.byref(p)))
        return p.value

    def stream(self):
        return lib().vmlm_decoder_stream(self._h)

    def time_gemv(self, which: int, iters: int):
        """Mean per-launch duration (us, HIP events on the session stream) of
        one decode-step GEMV over every layer in turn, and its algorithmic
        bytes. which: 0 qkv, 1 o, 2 gate/up, 3 down, 4 LM head; the kernels of
        the program the session runs (fused full-K or k-slice). On the k-slice
        program 5, 6, 7 time the o, gate/up or down projection together with
        the kernel that reduces its partials (also on the full-K program).
        8..11: a plain read of the q/k/v, o, gate/up or down weights; 12: the
        decode attention; 13: an empty kernel; 14, 15: the full-K q/k/v
        projection at four tiles per workgroup, the full-K gate/up at one tile
        pair. Launches are replayed from one HIP graph."""
        us = C.c_float()
        nbytes = C.c_double()
        check(lib().vmlm_decoder_time_gemv(self._h, int(which), int(iters), C.byref(us),
                                           C.byref(nbytes)))
        return us.value, nbytes.value
