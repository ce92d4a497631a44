"""Programs for the VM executor, in the instruction structure of the
reference's program builders:

* the MiniCPM-shaped decoder of tools/p12_build_minicpm.py: prefill of a
  token prompt (:455-530 embedding, :766-792 layer, :794-840 KV cache of the
  prompt, :990-994 final norm and LM head), optionally with its layers as a
  LAYERB / LOOP_CNT loop over one layer template (:700-760, :842-870);
* the unrolled greedy generation of tools/p14_gen_build.py:470-560 (each
  step: EMB of st_gen[k], the layer stack against the cached K/V, logits,
  TOPK_IDX fed back with WRITECOL into st_gen[k+1]);
* a step-looped generation (no reference counterpart): one decode step as a
  LOOP_CNT body whose RoPE position, cache column and softmax width come
  from slots (the executor's runtime-operand flags), instead of one
  unrolled copy per step with compile-time positions.

Token ids enter through the state slots st_tok [1,S] and st_gen [1,G+1]
(written by the caller before run(), as the reference runtime fills them
from tokens.bin / gen_tokens.bin). `weights` is the dict of
sparrow_amd.model.make_weights (int8 weights with per-row scales, bf16
embedding and LM head).
"""
from __future__ import annotations

import numpy as np

from . import vmb

LAYER_CONSTS = ("in_ln", "q", "k", "v", "o", "post_ln", "gate", "up", "down")
_W = dict(q=("wq", "sq"), k=("wk", "sk"), v=("wv", "sv"), o=("wo", "so"), gate=("wg", "sg"),
          up=("wu", "su"), down=("wd", "sd"))


def _emit_layer_consts(P, L, li, tag, scalars, cfg):
    """One layer's constants in a fixed order (uniform stride across layers):
    in_ln, q/q_sc, k/k_sc, v/v_sc, o/o_sc, post_ln, gate/.., up/.., down/..,
    then (looped programs) the layer's own eps/theta/scale scalars."""
    for name in LAYER_CONSTS:
        if name in ("in_ln", "post_ln"):
            P.const(f"{tag}_{name}", L[name].reshape(1, -1))
        else:
            w, s = _W[name]
            P.const(f"{tag}_{name}", L[w], "i8")
            P.const(f"{tag}_{name}_sc", L[s].reshape(-1, 1))
    if scalars:
        P.scalar(f"{tag}_eps1", cfg["eps"])
        P.scalar(f"{tag}_theta1", cfg["theta"])
        P.scalar(f"{tag}_scale1", cfg["attn_scale"])


def _gemm(P, dst, a, w):
    P.ins("GEMM", P[dst], P[a], P[w], dt=P[w + "_sc"])


def _layer(P, tag, S, cfg, s_eps, s_theta, s_scale):
    """tools/p12_build_minicpm.py:766-792: one layer of the prefill."""
    H, NH, HD = cfg["hidden"], cfg["n_heads"], cfg["head_dim"]
    P.ins("RMSNORM", P["xn"], P["h"], P[f"{tag}_in_ln"], dt=P[s_eps])
    for w in ("q", "k", "v"):
        _gemm(P, w, "xn", f"{tag}_{w}")
    for hh in range(NH):
        P.ins("SLICE", P["qh"], P["q"], hh * HD)
        P.ins("SLICE", P["kh"], P["k"], hh * HD)
        P.ins("SLICE", P["vh"], P["v"], hh * HD)
        P.ins("ROPE", P["qrot"], P["qh"], P[s_theta], dt=0)
        P.ins("ROPE", P["krot"], P["kh"], P[s_theta], dt=0)
        P.ins("GEMM", P["sc"], P["qrot"], P["krot"])
        P.ins("SCALE", P["sc"], P["sc"], P[s_scale])
        P.ins("SOFTMAX", P["sc"], P["sc"], fl=vmb.FL_CAUSAL)
        P.ins("GEMM", P["ctx"], P["sc"], P["vh"], fl=vmb.FL_TRANS_B)
        P.ins("WRITECOL", P["att"], P["ctx"], hh * HD)
    _gemm(P, "oproj", "att", f"{tag}_o")
    P.ins("EWADD", P["h2"], P["h"], P["oproj"])
    P.ins("RMSNORM", P["xn"], P["h2"], P[f"{tag}_post_ln"], dt=P[s_eps])
    _gemm(P, "gate", "xn", f"{tag}_gate")
    _gemm(P, "up", "xn", f"{tag}_up")
    P.ins("ACT", P["acts"], P["gate"], fl=vmb.ACT["silu"])
    P.ins("EWMUL", P["acts"], P["acts"], P["up"])
    _gemm(P, "down", "acts", f"{tag}_down")
    P.ins("EWADD", P["h"], P["h2"], P["down"])


def _cache_prompt(P, li, S, cfg):
    """tools/p12_build_minicpm.py:794-840: rotated K and raw V of the prompt
    positions into the per-head state caches st_kc / st_vc [HD, PMAX]."""
    HD = cfg["head_dim"]
    for hj in range(cfg["n_heads"]):
        P.ins("SLICE", P["kcraw"], P["k"], hj * HD)
        P.ins("ROPE", P["kcrot"], P["kcraw"], P["theta1"], dt=0)
        P.ins("SLICE", P["vcraw"], P["v"], hj * HD)
        P.ins("TRANSPOSE", P["kcrotT"], P["kcrot"])
        P.ins("TRANSPOSE", P["vcrawT"], P["vcraw"])
        for p in range(S):
            P.ins("SLICE", P["kcol"], P["kcrotT"], p)
            P.ins("WRITECOL", P[f"st_kc{li}_{hj}"], P["kcol"], p)
            P.ins("SLICE", P["vcol"], P["vcrawT"], p)
            P.ins("WRITECOL", P[f"st_vc{li}_{hj}"], P["vcol"], p)


def minicpm_program(cfg: dict, weights: dict, S: int, G: int = 0, looped: bool = False,
                    step_loop: bool = False, print_prefill: bool = True) -> vmb.Program:
    """The decoder program: prefill of S prompt tokens (st_tok), then G
    greedy steps (st_gen[0] = the caller's first token, normally the
    prefill's argmax; each step writes its argmax to st_gen[k+1]).

    looped: the prefill's layers as a LAYERB / LOOP_CNT loop over layer 0's
    constant names (prefill only, G must be 0, as in the reference builder).
    step_loop: the G steps as one LOOP_CNT body with runtime RoPE position,
    cache column and softmax width.
    PRINTs: the prefill's logits [S, V] (print_prefill), then per step its
    logits [1, V] and the token it read."""
    if looped and G:
        raise ValueError("looped layers cover the prefill only")
    H, NH, HD, I, V = cfg["hidden"], cfg["n_heads"], cfg["head_dim"], cfg["inter"], cfg["vocab"]
    NL = cfg["n_layers"]
    PMAX = S + G
    P = vmb.Program()
    # ---- constants: per-layer blocks first (uniform stride), then globals
    for li, L in enumerate(weights["layers"]):
        _emit_layer_consts(P, L, li, f"L{li}", looped, cfg)
    P.const("embed", weights["embed"], "bf16")
    P.const("lm_head", weights["lm_head"], "bf16")
    P.const("final_norm", weights["final_norm"].reshape(1, -1))
    P.scalar("eps1", cfg["eps"])
    P.scalar("theta1", cfg["theta"])
    P.scalar("scale1", cfg["attn_scale"])
    # ---- activation and state slots
    for name, r, c in (("h", S, H), ("xn", S, H), ("q", S, H), ("k", S, H), ("v", S, H),
                       ("qh", S, HD), ("kh", S, HD), ("vh", S, HD), ("qrot", S, HD),
                       ("krot", S, HD), ("sc", S, S), ("ctx", S, HD), ("att", S, H),
                       ("oproj", S, H), ("h2", S, H), ("gate", S, I), ("up", S, I),
                       ("acts", S, I), ("down", S, H), ("logits", S, V), ("hflat", S, H)):
        P.act(name, r, c)
    P.state("st_tok", 1, S)
    for i in range(S):
        P.act(f"tok{i}", 1, 1)
        P.act(f"e{i}", 1, H)
        P.act(f"hcat{i}", 1, H * (i + 1))
    # ---- h = embed[tokens] (p12:455-530): one EMB per token, rows chained
    for i in range(S):
        P.ins("SLICE", P[f"tok{i}"], P["st_tok"], i)
        P.ins("EMB", P[f"e{i}"], P["embed"], P[f"tok{i}"])
    P.ins("COPY", P["hcat0"], P["e0"])
    for i in range(1, S):
        P.ins("CONCAT", P[f"hcat{i}"], P[f"hcat{i - 1}"], P[f"e{i}"])
    P.ins("COPY", P["hflat"], P[f"hcat{S - 1}"])
    P.ins("COPY", P["h"], P["hflat"])
    if G:
        for name, r, c in (("kcraw", S, HD), ("kcrot", S, HD), ("vcraw", S, HD),
                           ("kcrotT", HD, S), ("vcrawT", HD, S), ("kcol", HD, 1),
                           ("vcol", HD, 1)):
            P.act(name, r, c)
        for li in range(NL):
            for hj in range(NH):
                P.state(f"st_kc{li}_{hj}", HD, PMAX)
                P.state(f"st_vc{li}_{hj}", HD, PMAX)
    # ---- layers
    if looped:
        stride = _layer_stride(P, NL)
        P.act("lcnt", 1, 1)
        P.act("lstride", 1, 1)
        P.act("lnl", 1, 1)
        P.act("lneg", 1, 1)
        P.scalar("layer_stride", float(stride))
        P.scalar("layer_count", float(NL))
        P.scalar("neg_layer_count", float(-NL))
        P.ins("COPY", P["lcnt"], P["layer_count"])
        P.ins("COPY", P["lstride"], P["layer_stride"])
        P.ins("COPY", P["lnl"], P["neg_layer_count"])
        top = P.label()
        _layer(P, "L0", S, cfg, "L0_eps1", "L0_theta1", "L0_scale1")
        P.ins("LAYERB", 0, P["lstride"])
        P.ins("LOOP_CNT", top, P["lcnt"])
        P.ins("EWMUL", P["lneg"], P["lstride"], P["lnl"])
        P.ins("LAYERB", 0, P["lneg"])
    else:
        for li in range(NL):
            _layer(P, f"L{li}", S, cfg, "eps1", "theta1", "scale1")
            if G:
                _cache_prompt(P, li, S, cfg)
    P.ins("RMSNORM", P["xn"], P["h"], P["final_norm"], dt=P["eps1"])
    P.ins("GEMM", P["logits"], P["xn"], P["lm_head"])
    if print_prefill:
        P.ins("PRINT", P["logits"])
    if G:
        (_decode_loop if step_loop else _decode_unrolled)(P, cfg, S, G)
    P.ins("HALT")
    return P


def _layer_stride(P, NL):
    """Bytes between layer l's constants and layer l+1's (the same for
    every constant of the layer, as LAYERB requires)."""
    off, pos = {}, 0
    for c in P.consts:
        off[c.name] = pos
        pos += (len(c.data) + 63) // 64 * 64
    strides = {off[f"L{l + 1}_{n}"] - off[f"L{l}_{n}"] for l in range(NL - 1)
               for n in ("in_ln", "q", "down_sc", "scale1")}
    if len(strides) > 1:
        raise ValueError(f"per-layer constants are not uniformly strided: {strides}")
    return strides.pop() if strides else 0


def _decode_slots(P, cfg, S, G):
    H, NH, HD, I, V = cfg["hidden"], cfg["n_heads"], cfg["head_dim"], cfg["inter"], cfg["vocab"]
    P.state("st_gen", 1, G + 1)
    for name, r, c in (("gtok", 1, 1), ("eh", 1, H), ("hdec", 1, H), ("xnd", 1, H),
                       ("qd", 1, H), ("kd", 1, H), ("vd", 1, H), ("qdh", 1, HD),
                       ("kdh", 1, HD), ("vdh", 1, HD), ("kdrot", 1, HD), ("qdrot", 1, HD),
                       ("kdT", HD, 1), ("vdT", HD, 1), ("attd", 1, H), ("oprojd", 1, H),
                       ("h2d", 1, H), ("gated", 1, I), ("upd", 1, I), ("actsd", 1, I),
                       ("downd", 1, H), ("ctxd", 1, HD), ("nxt", 1, 1)):
        P.act(name, r, c)


def _decode_layer_tail(P, li):
    _gemm(P, "oprojd", "attd", f"L{li}_o")
    P.ins("EWADD", P["h2d"], P["hdec"], P["oprojd"])
    P.ins("RMSNORM", P["xnd"], P["h2d"], P[f"L{li}_post_ln"], dt=P["eps1"])
    _gemm(P, "gated", "xnd", f"L{li}_gate")
    _gemm(P, "upd", "xnd", f"L{li}_up")
    P.ins("ACT", P["actsd"], P["gated"], fl=vmb.ACT["silu"])
    P.ins("EWMUL", P["actsd"], P["actsd"], P["upd"])
    _gemm(P, "downd", "actsd", f"L{li}_down")
    P.ins("EWADD", P["hdec"], P["h2d"], P["downd"])


def _decode_unrolled(P, cfg, S, G):
    """tools/p14_gen_build.py:470-560, argmax sampler."""
    NL, NH, HD, V = cfg["n_layers"], cfg["n_heads"], cfg["head_dim"], cfg["vocab"]
    _decode_slots(P, cfg, S, G)
    for step in range(G):
        pos, live = S + step, S + step + 1
        P.act(f"kcv{step}", HD, live)
        P.act(f"vcv{step}", HD, live)
        P.act(f"scd{step}", 1, live)
        P.act(f"logitsd{step}", 1, V)
        P.ins("SLICE", P["gtok"], P["st_gen"], step)
        P.ins("EMB", P["eh"], P["embed"], P["gtok"])
        P.ins("COPY", P["hdec"], P["eh"])
        for li in range(NL):
            P.ins("RMSNORM", P["xnd"], P["hdec"], P[f"L{li}_in_ln"], dt=P["eps1"])
            for w in ("q", "k", "v"):
                _gemm(P, w + "d", "xnd", f"L{li}_{w}")
            for hj in range(NH):
                P.ins("SLICE", P["kdh"], P["kd"], hj * HD)
                P.ins("SLICE", P["vdh"], P["vd"], hj * HD)
                P.ins("ROPE", P["kdrot"], P["kdh"], P["theta1"], dt=pos)
                P.ins("TRANSPOSE", P["kdT"], P["kdrot"])
                P.ins("TRANSPOSE", P["vdT"], P["vdh"])
                P.ins("WRITECOL", P[f"st_kc{li}_{hj}"], P["kdT"], pos)
                P.ins("WRITECOL", P[f"st_vc{li}_{hj}"], P["vdT"], pos)
            for hh in range(NH):
                P.ins("SLICE", P["qdh"], P["qd"], hh * HD)
                P.ins("ROPE", P["qdrot"], P["qdh"], P["theta1"], dt=pos)
                P.ins("SLICE", P[f"kcv{step}"], P[f"st_kc{li}_{hh}"], 0)
                P.ins("SLICE", P[f"vcv{step}"], P[f"st_vc{li}_{hh}"], 0)
                P.ins("GEMM", P[f"scd{step}"], P["qdrot"], P[f"kcv{step}"], fl=vmb.FL_TRANS_B)
                P.ins("SCALE", P[f"scd{step}"], P[f"scd{step}"], P["scale1"])
                P.ins("SOFTMAX", P[f"scd{step}"], P[f"scd{step}"])
                P.ins("GEMM", P["ctxd"], P[f"scd{step}"], P[f"vcv{step}"])
                P.ins("WRITECOL", P["attd"], P["ctxd"], hh * HD)
            _decode_layer_tail(P, li)
        P.ins("RMSNORM", P["xnd"], P["hdec"], P["final_norm"], dt=P["eps1"])
        P.ins("GEMM", P[f"logitsd{step}"], P["xnd"], P["lm_head"])
        P.ins("PRINT", P[f"logitsd{step}"])
        P.ins("TOPK_IDX", P["nxt"], P[f"logitsd{step}"])
        P.ins("WRITECOL", P["st_gen"], P["nxt"], step + 1)


def _decode_loop(P, cfg, S, G):
    """The G steps as one LOOP_CNT body: the position, the cache column and
    the live width are slots advanced every step; scores and context run
    over the whole cache width [HD, S+G] with the softmax limited to the
    live positions (columns past them are 0 and the cache is zero there)."""
    NL, NH, HD, V = cfg["n_layers"], cfg["n_heads"], cfg["head_dim"], cfg["vocab"]
    PMAX = S + G
    _decode_slots(P, cfg, S, G)
    P.act("scd", 1, PMAX)
    P.act("logitsd", 1, V)
    for name in ("posf", "livef", "genc", "stepc"):
        P.act(name, 1, 1)
    P.scalar("one", 1.0)
    P.scalar("pos_init", float(S))
    P.scalar("live_init", float(S + 1))
    P.scalar("steps", float(G))
    P.ins("COPY", P["posf"], P["pos_init"])
    P.ins("COPY", P["livef"], P["live_init"])
    P.ins("COPY", P["genc"], P["one"])
    P.ins("COPY", P["stepc"], P["steps"])
    P.ins("SLICE", P["gtok"], P["st_gen"], 0)
    top = P.label()
    P.ins("EMB", P["eh"], P["embed"], P["gtok"])
    P.ins("COPY", P["hdec"], P["eh"])
    rt = 1 << 6
    for li in range(NL):
        P.ins("RMSNORM", P["xnd"], P["hdec"], P[f"L{li}_in_ln"], dt=P["eps1"])
        for w in ("q", "k", "v"):
            _gemm(P, w + "d", "xnd", f"L{li}_{w}")
        for hj in range(NH):
            P.ins("SLICE", P["kdh"], P["kd"], hj * HD)
            P.ins("SLICE", P["vdh"], P["vd"], hj * HD)
            P.ins("ROPE", P["kdrot"], P["kdh"], P["theta1"], dt=P["posf"], fl=rt)
            P.ins("TRANSPOSE", P["kdT"], P["kdrot"])
            P.ins("TRANSPOSE", P["vdT"], P["vdh"])
            P.ins("WRITECOL", P[f"st_kc{li}_{hj}"], P["kdT"], 0, dt=P["posf"], fl=rt)
            P.ins("WRITECOL", P[f"st_vc{li}_{hj}"], P["vdT"], 0, dt=P["posf"], fl=rt)
        for hh in range(NH):
            P.ins("SLICE", P["qdh"], P["qd"], hh * HD)
            P.ins("ROPE", P["qdrot"], P["qdh"], P["theta1"], dt=P["posf"], fl=rt)
            P.ins("GEMM", P["scd"], P["qdrot"], P[f"st_kc{li}_{hh}"], fl=vmb.FL_TRANS_B)
            P.ins("SCALE", P["scd"], P["scd"], P["scale1"])
            P.ins("SOFTMAX", P["scd"], P["scd"], P["livef"], fl=rt)
            P.ins("GEMM", P["ctxd"], P["scd"], P[f"st_vc{li}_{hh}"])
            P.ins("WRITECOL", P["attd"], P["ctxd"], hh * HD)
        _decode_layer_tail(P, li)
    P.ins("RMSNORM", P["xnd"], P["hdec"], P["final_norm"], dt=P["eps1"])
    P.ins("GEMM", P["logitsd"], P["xnd"], P["lm_head"])
    P.ins("PRINT", P["logitsd"])
    P.ins("TOPK_IDX", P["nxt"], P["logitsd"])
    P.ins("WRITECOL", P["st_gen"], P["nxt"], 0, dt=P["genc"], fl=rt)
    P.ins("COPY", P["gtok"], P["nxt"])
    P.ins("EWADD", P["posf"], P["posf"], P["one"])
    P.ins("EWADD", P["livef"], P["livef"], P["one"])
    P.ins("EWADD", P["genc"], P["genc"], P["one"])
    P.ins("LOOP_CNT", top, P["stepc"])
