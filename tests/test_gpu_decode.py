"""The GPU int8 decode path against the CPU oracle: logits position by
position on a small model, identical greedy token streams on the small
model and on BASELINE config 4 (against the committed oracle fixture)."""

import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from tests.conftest import announce
from vx_amd.decode import LlamaI8
from vx_amd.llama import CONFIG_DECODE, CONFIG_TINY, LlamaConfig, make_model, make_prompt

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "decode_config4.json"


def assert_same_tokens(got, want, margin):
    """Identical greedy streams; a disagreement is reported with the logit
    margin the oracle had at that step."""
    got, want = list(map(int, got)), list(map(int, want))
    if got != want:
        i = next(k for k in range(len(want)) if got[k] != want[k])
        raise AssertionError(f"token {i}: gpu {got[i]} vs oracle {want[i]} "
                             f"(oracle margin there {margin[i]:.3g})")


@pytest.mark.parametrize("cfg", [CONFIG_TINY,
                                 LlamaConfig(dim=128, hidden_dim=256, n_layers=3, n_heads=2,
                                             n_kv_heads=1, vocab_size=512, seq_len=96),
                                 # rows wider than 1024 and 2048 columns (the GEMVs built for
                                 # 2 and 4 column segments), grouped KV heads
                                 LlamaConfig(dim=1152, hidden_dim=3072, n_layers=1, n_heads=18,
                                             n_kv_heads=6, vocab_size=512, seq_len=64),
                                 # head size 128
                                 LlamaConfig(dim=1024, hidden_dim=2816, n_layers=1, n_heads=8,
                                             n_kv_heads=8, vocab_size=384, seq_len=48),
                                 # a cache length that the attention split does not divide,
                                 # filled to its last row
                                 LlamaConfig(dim=96, hidden_dim=160, n_layers=2, n_heads=3,
                                             n_kv_heads=1, vocab_size=200, seq_len=37)])
def test_logits_per_position_match_oracle(hiplib, cfg):
    announce(f"decode logits {cfg}")
    weights = make_model(cfg, seed=3)
    tokens = list(make_prompt(cfg, n=cfg.seq_len if cfg.seq_len < 40 else 20, seed=5))
    model = LlamaI8(hiplib, cfg, weights)
    got = model.logits(tokens)
    model.close()
    kv = np.zeros(2 * cfg.n_layers * cfg.seq_len * cfg.kv_dim, np.float32)
    for pos, tok in enumerate(tokens):
        want = oracle.llama_forward(cfg.as_dict(), weights, kv, int(tok), pos)
        scale = float(np.abs(want).max())
        err = float(np.abs(got[pos] - want).max())
        assert err <= 1e-3 * scale + 1e-5, f"position {pos}: max abs error {err} (scale {scale})"


@pytest.mark.parametrize("graph", [True, False])
def test_tiny_greedy_stream_matches_oracle(hiplib, graph):
    announce(f"decode tiny greedy graph={graph}")
    cfg = CONFIG_TINY
    weights = make_model(cfg, seed=3)
    prompt = make_prompt(cfg, n=6, seed=5)
    want, margin = oracle.llama_generate(cfg.as_dict(), weights, prompt, 40)
    model = LlamaI8(hiplib, cfg, weights)
    got, gm = model.generate(prompt, 40, graph=graph)
    model.close()
    assert_same_tokens(got, want, margin)
    np.testing.assert_allclose(gm, margin, atol=1e-3)


@pytest.mark.parametrize("cfg", [
    # layer 0's token choice built for 2 and 4 column segments (rows of 1152 and 2304)
    LlamaConfig(dim=1152, hidden_dim=3072, n_layers=1, n_heads=18, n_kv_heads=6,
                vocab_size=512, seq_len=64),
    LlamaConfig(dim=2304, hidden_dim=1024, n_layers=1, n_heads=18, n_kv_heads=6,
                vocab_size=640, seq_len=48)])
def test_wide_rows_greedy_stream_matches_oracle(hiplib, cfg):
    announce(f"decode wide greedy {cfg}")
    weights = make_model(cfg, seed=3)
    prompt = make_prompt(cfg, n=5, seed=5)
    want, margin = oracle.llama_generate(cfg.as_dict(), weights, prompt, 30)
    model = LlamaI8(hiplib, cfg, weights)
    got, gm = model.generate(prompt, 30)
    model.close()
    assert_same_tokens(got, want, margin)
    np.testing.assert_allclose(gm, margin, atol=1e-3)


@pytest.mark.parametrize("n_prompt", [1, 6])
def test_single_step_and_single_token_prompt(hiplib, n_prompt):
    """One step: the only token is the one recorded after the last prompt
    position; a one-token prompt: the first step already reads candidates
    (position 1 on)."""
    announce(f"decode one step, prompt {n_prompt}")
    cfg = CONFIG_TINY
    weights = make_model(cfg, seed=3)
    prompt = make_prompt(cfg, n=n_prompt, seed=5)
    want, margin = oracle.llama_generate(cfg.as_dict(), weights, prompt, 8)
    model = LlamaI8(hiplib, cfg, weights)
    for graph in (True, False):
        got, gm = model.generate(prompt, 1, graph=graph)
        assert int(got[0]) == int(want[0]), f"graph={graph}"
        np.testing.assert_allclose(gm[:1], margin[:1], atol=1e-3)
        got, gm = model.generate(prompt, 8, graph=graph)
        assert_same_tokens(got, want, margin)
    model.close()


@pytest.mark.parametrize("graph", [True, False])
def test_large_vocab_greedy_stream_matches_oracle(hiplib, graph):
    """A vocabulary of 40000 leaves 1250 classifier candidates, more than the
    1024 that layer 0's token choice requests before its weights: the rest
    go through its second loop. The prompt ends on token 39001, so the
    first choices are won by a row that only those candidates cover."""
    announce(f"decode vocab 40000 greedy graph={graph}")
    cfg = LlamaConfig(dim=64, hidden_dim=128, n_layers=2, n_heads=4, n_kv_heads=2,
                      vocab_size=40000, seq_len=64)
    weights = make_model(cfg, seed=3)
    prompt = make_prompt(cfg, n=6, seed=5)
    prompt[-1] = 39001
    want, margin = oracle.llama_generate(cfg.as_dict(), weights, prompt, 40)
    assert any(int(t) >= 32768 for t in want)  # rows of candidates 1024 and up
    model = LlamaI8(hiplib, cfg, weights)
    got, gm = model.generate(prompt, 40, graph=graph)
    model.close()
    assert_same_tokens(got, want, margin)
    np.testing.assert_allclose(gm, margin, atol=1e-3)


def test_config4_greedy_stream_matches_oracle(hiplib):
    """BASELINE config 4, 16-token prompt, 256 greedy tokens: the same stream
    as the CPU oracle (tests/golden/make_decode_golden.py)."""
    announce("decode config 4 greedy 256")
    g = json.loads(GOLDEN.read_text())
    cfg = CONFIG_DECODE
    assert g["config"] == cfg.as_dict()
    weights = make_model(cfg, seed=g["model_seed"])
    prompt = make_prompt(cfg, n=16, seed=g["prompt_seed"])
    assert list(map(int, prompt)) == g["prompt"]
    model = LlamaI8(hiplib, cfg, weights)
    got, gm = model.generate(prompt, g["n_steps"])
    again, _ = model.generate(prompt, g["n_steps"])
    model.close()
    assert np.array_equal(got, again), "two runs of the same generation differ"
    assert_same_tokens(got, g["tokens"], g["margins"])
    np.testing.assert_allclose(gm, g["margins"], atol=2e-4)
    # logits at the probed positions of the same sequence
    model = LlamaI8(hiplib, cfg, weights)
    seq = g["prompt"] + g["tokens"][:-1]
    logits = model.logits(seq)
    model.close()
    for pos, probe in g["logit_probes"].items():
        row = logits[int(pos)]
        assert list(np.argsort(-row, kind="stable")[:4]) == probe["index"][:4], f"position {pos}"
        np.testing.assert_allclose(row[probe["index"]], probe["value"], atol=2e-4,
                                   err_msg=f"position {pos}")
    # every position: mean and spread of all 32000 logits (a wrong term
    # anywhere in the vocabulary moves them; GPU and oracle logits differ by
    # a few 1e-6 from summation order)
    l64 = logits.astype(np.float64)
    moments = np.stack([l64.mean(axis=1), l64.std(axis=1)], axis=1)
    np.testing.assert_allclose(moments, np.array(g["logit_moments"]), atol=2e-5,
                               err_msg="logit mean/std per position")


def test_refusals(hiplib):
    announce("decode refusals")
    cfg = LlamaConfig(dim=96, hidden_dim=128, n_layers=1, n_heads=5, n_kv_heads=5,
                      vocab_size=64, seq_len=16)  # dim not a multiple of n_heads
    with pytest.raises(RuntimeError):
        LlamaI8(hiplib, cfg, make_model(CONFIG_TINY, seed=0))
    model = LlamaI8(hiplib, CONFIG_TINY, make_model(CONFIG_TINY, seed=0))
    with pytest.raises(RuntimeError):
        model.generate([1, 2, 3], CONFIG_TINY.seq_len)  # past seq_len
    with pytest.raises(RuntimeError):
        model.generate([CONFIG_TINY.vocab_size], 4)  # token outside the vocabulary
    model.close()


def test_model_read_from_checkpoint_file_generates_like_oracle(hiplib, tmp_path):
    """A llama2.c checkpoint read through vx_llama_i8_read (quantized on the
    way in), uploaded and run greedily, against the oracle on the same
    weights; the VXQ8 file saved from it runs identically."""
    from tests.test_llama_io import f32_model
    from vx_amd.decode import read_model, save_model, write_checkpoint

    announce("decode from a checkpoint file")
    cfg = CONFIG_TINY
    write_checkpoint(tmp_path / "tiny.bin", cfg, f32_model(cfg, seed=21))
    rcfg, weights = read_model(hiplib, tmp_path / "tiny.bin")
    assert rcfg == cfg
    prompt = make_prompt(cfg, n=5, seed=8)
    want, margin = oracle.llama_generate(cfg.as_dict(), weights, prompt, 30)
    model = LlamaI8(hiplib, cfg, weights)
    got, _ = model.generate(prompt, 30)
    model.close()
    assert_same_tokens(got, want, margin)
    save_model(hiplib, tmp_path / "tiny.q8", cfg, weights)
    _, again = read_model(hiplib, tmp_path / "tiny.q8")
    model = LlamaI8(hiplib, cfg, again)
    got2, _ = model.generate(prompt, 30)
    model.close()
    assert list(map(int, got2)) == list(map(int, got))


@pytest.mark.parametrize("cfg,n", [
    # head size 256: a split's rounds hold 32 positions, so 150 positions take two
    (LlamaConfig(dim=512, hidden_dim=256, n_layers=1, n_heads=2, n_kv_heads=1,
                 vocab_size=256, seq_len=160), 150),
    # head size 64 (config 4's): rounds of 128 per split, 560 positions take two
    (LlamaConfig(dim=128, hidden_dim=256, n_layers=1, n_heads=2, n_kv_heads=2,
                 vocab_size=256, seq_len=576), 560)])
def test_long_sequence_logits_match_oracle(hiplib, cfg, n):
    """Caches long enough that each attention workgroup rescales its running
    softmax between rounds of key and value rows."""
    announce(f"decode long logits {cfg} n={n}")
    weights = make_model(cfg, seed=4)
    tokens = list(make_prompt(cfg, n=n, seed=6))
    model = LlamaI8(hiplib, cfg, weights)
    got = model.logits(tokens)
    model.close()
    kv = np.zeros(2 * cfg.n_layers * cfg.seq_len * cfg.kv_dim, np.float32)
    for pos, tok in enumerate(tokens):
        want = oracle.llama_forward(cfg.as_dict(), weights, kv, int(tok), pos)
        scale = float(np.abs(want).max())
        err = float(np.abs(got[pos] - want).max())
        assert err <= 1e-3 * scale + 1e-5, f"position {pos}: max abs error {err} (scale {scale})"
