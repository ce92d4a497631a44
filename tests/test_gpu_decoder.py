"""GPU parity of the MiniCPM-shaped decoder session against the CPU oracle's
run of the same program (tools/p12_build_minicpm.py + p14_gen_build.py).

Bars: greedy token chains identical; logits within 1e-4 of their RMS;
batch-16 sequences bitwise equal to the same sequences decoded alone."""
import sys
import time

import numpy as np
import pytest

from sparrow_amd import model as M

pytestmark = pytest.mark.gpu


def rms(x):
    return float(np.sqrt(np.mean(np.asarray(x, np.float64) ** 2)))


def log(msg):
    print(msg, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def tiny():
    cfg = M.tiny_config(n_layers=3, hidden=256, n_heads=4, inter=512, vocab=3000)
    return cfg, M.make_weights(cfg, seed=11)


def test_tiny_generate_matches_oracle(hip, oracle, tiny):
    from sparrow_amd.decoder import Decoder
    cfg, W = tiny
    prompts = M.make_prompts(cfg, 2, 20, seed=5)
    with Decoder(cfg, batch=2, cap=64) as dec:
        dec.load(W)
        t0, logits = dec.prefill(prompts, want_logits=True)
        toks, last = dec.decode(24, want_logits=True)
    for b in range(2):
        ref = oracle.DecoderOracle(W, cfg, cap=64)
        rl, _ = ref.prefill(prompts[b])
        assert np.abs(logits[b] - rl).max() <= 1e-4 * rms(rl)
        ref2 = oracle.DecoderOracle(W, cfg, cap=64)
        chain, margins = ref2.generate(prompts[b], 24)
        got = np.concatenate([[t0[b]], toks[:, b]])
        log(f"seq {b}: min top1-top2 margin {margins.min():.3e}")
        assert np.array_equal(got, chain)


@pytest.mark.parametrize("batch", [1, 3, 5])
def test_tiny_fused_matches_kslice_and_oracle(hip, oracle, tiny, batch):
    """The fused five-launch layer (default at batch <= 5) against the
    k-slice eight-launch program and the oracle: logits within 1e-4 of
    their RMS, identical greedy chains."""
    from sparrow_amd.decoder import Decoder
    cfg, W = tiny
    prompts = M.make_prompts(cfg, batch, 13, seed=21)
    out = {}
    for fused in (True, False):
        with Decoder(cfg, batch=batch, cap=64) as dec:
            assert dec.fused  # the default at this batch
            dec.load(W)
            dec.set_fused(fused)
            assert dec.fused == fused
            t0, _ = dec.prefill(prompts)
            toks, last = dec.decode(16, want_logits=True)
        out[fused] = (np.concatenate([t0[None, :], toks], 0), last)
    assert np.array_equal(out[True][0], out[False][0])
    for b in range(batch):
        ref = oracle.DecoderOracle(W, cfg, cap=64)
        chain, _ = ref.generate(prompts[b], 16)
        assert np.array_equal(out[True][0][:, b], chain)
        # the oracle's logits of the last step: prefill, then 16 steps fed
        # with the chain's tokens
        ref = oracle.DecoderOracle(W, cfg, cap=64)
        ref.prefill(prompts[b])
        for i in range(16):
            lr, _ = ref.step(chain[i], 13 + i)
        assert np.abs(out[True][1][b] - lr).max() <= 1e-4 * rms(lr)
        assert np.abs(out[False][1][b] - lr).max() <= 1e-4 * rms(lr)


def test_tiny_batch16_kslice_matches_oracle(hip, oracle, tiny):
    """Batch 16 (the k-slice program): every sequence's chain equals the
    oracle's, and the last step's logits are within 1e-4 of their RMS."""
    from sparrow_amd.decoder import Decoder
    cfg, W = tiny
    prompts = M.make_prompts(cfg, 16, 7, seed=31)
    with Decoder(cfg, batch=16, cap=64) as dec:
        assert not dec.fused
        dec.load(W)
        t0, _ = dec.prefill(prompts)
        toks, last = dec.decode(6, want_logits=True)
    got = np.concatenate([t0[None, :], toks], 0)
    for b in (0, 5, 15):
        ref = oracle.DecoderOracle(W, cfg, cap=64)
        chain, _ = ref.generate(prompts[b], 6)
        assert np.array_equal(got[:, b], chain)
        ref = oracle.DecoderOracle(W, cfg, cap=64)
        ref.prefill(prompts[b])
        for i in range(6):
            lr, _ = ref.step(chain[i], 7 + i)
        assert np.abs(last[b] - lr).max() <= 1e-4 * rms(lr)


@pytest.fixture(scope="module")
def small768():
    cfg = M.tiny_config(n_layers=2, hidden=768, n_heads=12, inter=2048, vocab=3000)
    return cfg, M.make_weights(cfg, seed=13)


@pytest.mark.parametrize("batch", [16, 7])
def test_fullk_matches_kslice_and_oracle(hip, oracle, small768, batch):
    """The full-K program (the default from batch 6 at hidden 768..2304: q/k/v
    and gate/up in one launch each, SiLU * up in the epilogue, down over
    f32 rows quantized while staged) against the k-slice program and the
    oracle: identical greedy chains, last-step logits within 1e-4 of their
    RMS, at a full and a ragged batch."""
    from sparrow_amd.decoder import Decoder
    cfg, W = small768
    prompts = M.make_prompts(cfg, batch, 11, seed=41)
    out = {}
    for prog in (Decoder.FULLK, Decoder.KSLICE):
        with Decoder(cfg, batch=batch, cap=64) as dec:
            assert dec.program == Decoder.FULLK
            dec.load(W)
            dec.set_program(prog)
            assert dec.program == prog
            t0, _ = dec.prefill(prompts)
            toks, last = dec.decode(8, want_logits=True)
        out[prog] = (np.concatenate([t0[None, :], toks], 0), last)
    assert np.array_equal(out[Decoder.FULLK][0], out[Decoder.KSLICE][0])
    for b in (0, batch // 2, batch - 1):
        ref = oracle.DecoderOracle(W, cfg, cap=64)
        chain, _ = ref.generate(prompts[b], 8)
        assert np.array_equal(out[Decoder.FULLK][0][:, b], chain)
        ref = oracle.DecoderOracle(W, cfg, cap=64)
        ref.prefill(prompts[b])
        for i in range(8):
            lr, _ = ref.step(chain[i], 11 + i)
        for prog in out:
            assert np.abs(out[prog][1][b] - lr).max() <= 1e-4 * rms(lr), (prog, b)


def test_fullk_graph_equals_eager(hip, small768):
    """The full-K step replayed from its HIP graph gives the eager launches'
    logits bitwise."""
    from sparrow_amd.decoder import Decoder
    cfg, W = small768
    prompts = M.make_prompts(cfg, 9, 6, seed=8)
    out = []
    for graph in (True, False):
        with Decoder(cfg, batch=9, cap=32) as dec:
            dec.load(W)
            dec.set_graph(graph)
            dec.prefill(prompts)
            toks, logits = dec.decode(5, want_logits=True)
            out.append((toks, logits))
    assert np.array_equal(out[0][0], out[1][0])
    assert np.array_equal(out[0][1].view(np.uint32), out[1][1].view(np.uint32))


def test_fused_guard(hip, tiny):
    from sparrow_amd import VmlmError
    from sparrow_amd.decoder import Decoder
    cfg, W = tiny
    with Decoder(cfg, batch=6, cap=64) as dec:
        assert not dec.fused
        with pytest.raises(VmlmError):
            dec.set_fused(True)


def test_tiny_graph_equals_eager(hip, tiny):
    from sparrow_amd.decoder import Decoder
    cfg, W = tiny
    prompts = M.make_prompts(cfg, 1, 9, seed=6)
    out = []
    for graph in (True, False):
        with Decoder(cfg, batch=1, cap=64) as dec:
            dec.load(W)
            dec.set_graph(graph)
            dec.prefill(prompts)
            toks, logits = dec.decode(12, want_logits=True)
            out.append((toks, logits))
    assert np.array_equal(out[0][0], out[1][0])
    assert np.array_equal(out[0][1].view(np.uint32), out[1][1].view(np.uint32))


def test_tiny_guards(hip, tiny):
    from sparrow_amd import VmlmError
    from sparrow_amd.decoder import Decoder
    cfg, W = tiny
    with Decoder(cfg, batch=1, cap=16) as dec:
        dec.load(W)
        with pytest.raises(VmlmError) as e:
            dec.prefill(np.array([[1, 2, cfg["vocab"]]], np.int32))  # id == vocab
        assert e.value.code == 9
        dec.prefill(np.array([[1, 2, 3]], np.int32))
        with pytest.raises(VmlmError) as e:
            dec.decode(14)  # would write position 16 == cap
        assert e.value.code == 9


@pytest.fixture(scope="module")
def minicpm():
    t = time.time()
    cfg = M.minicpm_2b_config()
    W = M.make_weights(cfg, seed=3)
    log(f"MiniCPM-2B-shape weights generated in {time.time() - t:.1f}s")
    return cfg, W


def test_minicpm_batch1_64_greedy_tokens_identical(hip, oracle, minicpm):
    """prompt of 128 ids, greedy 64 steps at batch 1,
    token chain identical to the CPU oracle's."""
    from sparrow_amd.decoder import Decoder
    cfg, W = minicpm
    prompt = M.make_prompts(cfg, 1, 128, seed=3)
    t = time.time()
    with Decoder(cfg, batch=1, cap=256) as dec:
        dec.load(W)
        t0, logits = dec.prefill(prompt, want_logits=True)
        toks, _ = dec.decode(64)
    got = np.concatenate([t0, toks[:, 0]])
    log(f"GPU prefill+64 steps done in {time.time() - t:.1f}s")
    t = time.time()
    ref = oracle.DecoderOracle(W, cfg, cap=256)
    chain, margins = ref.generate(prompt[0], 64)
    log(f"oracle chain in {time.time() - t:.1f}s; min margin {margins.min():.3e}")
    assert np.array_equal(got, chain), f"first divergence at {np.argmax(got != chain)}"


@pytest.mark.parametrize("program", [2, 0])
def test_minicpm_batch16_64_greedy_tokens_identical(hip, oracle, minicpm, golden_dir, program):
    """BASELINE config 3 at batch 16: 16 prompts of 128 ids, 64 greedy steps
    on the full-K program (the default) and on the k-slice program. Every
    sequence's 65 tokens equal the CPU oracle's chain
    (tests/golden/minicpm2b_b16_chains.npz, written by make_decoder_chains.py
    from oracle.DecoderOracle.generate); for sequences 0 and 15 the oracle
    runs here as well, fed the chain, and the last step's logits are within
    1e-4 of their RMS."""
    from sparrow_amd.decoder import Decoder
    cfg, W = minicpm
    gold = np.load(golden_dir / "minicpm2b_b16_chains.npz")
    prompts = M.make_prompts(cfg, 16, 128, seed=3)
    assert np.array_equal(prompts, gold["prompts"])
    t = time.time()
    with Decoder(cfg, batch=16, cap=200) as dec:
        assert dec.program == Decoder.FULLK
        dec.load(W)
        dec.set_program(program)
        t0, _ = dec.prefill(prompts)
        toks, last = dec.decode(64, want_logits=True)
    got = np.concatenate([t0[None, :], toks], 0).T
    log(f"GPU batch-16 prefill+64 steps in {time.time() - t:.1f}s; "
        f"min oracle margin {gold['margins'].min():.3e}")
    for b in range(16):
        assert np.array_equal(got[b], gold["tokens"][b]), \
            f"sequence {b}: first divergence at {np.argmax(got[b] != gold['tokens'][b])}"
    for b in (0, 15):
        t = time.time()
        ref = oracle.DecoderOracle(W, cfg, cap=200)
        ref.prefill(prompts[b])
        for i in range(64):
            lr, _ = ref.step(gold["tokens"][b, i], 128 + i)
        log(f"oracle logits of sequence {b} in {time.time() - t:.1f}s")
        assert np.abs(last[b] - lr).max() <= 1e-4 * rms(lr)


def test_minicpm_batch16_equals_batch1(hip, minicpm):
    """Batch-16 decode: each sequence's chain is bitwise the chain it gets
    alone (rows never mix), checked for sequences 0 and 9 over 8 steps."""
    from sparrow_amd.decoder import Decoder
    cfg, W = minicpm
    prompts = M.make_prompts(cfg, 16, 128, seed=3)
    with Decoder(cfg, batch=16, cap=160) as dec:
        dec.load(W)
        chains = dec.generate(prompts, 8)
    for b in (0, 9):
        with Decoder(cfg, batch=1, cap=160) as dec:
            dec.load(W)
            alone = dec.generate(prompts[b:b + 1], 8)
        assert np.array_equal(chains[b], alone[0])


def test_time_gemv_follows_program(hip, tiny):
    """time_gemv times the launches of the program the session runs: on the
    fused program the o projection's bytes include the residual rows its
    epilogue reads (4 * batch * hidden more than the k-slice kernel's)."""
    from sparrow_amd.decoder import Decoder
    cfg, W = tiny
    with Decoder(cfg, batch=1, cap=64) as dec:
        dec.load(W)
        dec.prefill(M.make_prompts(cfg, 1, 5, seed=2))
        assert dec.fused
        us_f, b_f = dec.time_gemv(1, 4)
        dec.set_fused(False)
        us_k, b_k = dec.time_gemv(1, 4)
    assert us_f > 0 and us_k > 0
    assert b_f - b_k == 4 * 1 * cfg["hidden"]
