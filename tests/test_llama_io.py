"""Model files for the int8 decode path (vx_llama_i8_read / _save): the
reference's llama2.c checkpoint layout, quantized on the way in, and the
build's VXQ8 int8 file. Host-side only: runs without a GPU."""

import numpy as np
import pytest

import oracle
from vx_amd import llama
from vx_amd.decode import read_model, save_model, write_checkpoint
from vx_amd.runtime import DispatchLibrary

CFG = llama.CONFIG_TINY


@pytest.fixture(scope="module")
def lib():
    return DispatchLibrary(hip=True)


def f32_model(cfg, seed=5):
    rng = np.random.default_rng(seed)
    d, h, kv, L = cfg.dim, cfg.hidden_dim, cfg.kv_dim, cfg.n_layers

    def mat(*shape):
        return (rng.standard_normal(shape) * 0.02).astype(np.float32)

    m = {"tok": mat(cfg.vocab_size, d), "wq": mat(L, d, d), "wk": mat(L, kv, d),
         "wv": mat(L, kv, d), "wo": mat(L, d, d), "w1": mat(L, h, d), "w2": mat(L, d, h),
         "w3": mat(L, h, d)}
    m["rms_att"] = rng.uniform(0.5, 1.5, (L, d)).astype(np.float32)
    m["rms_ffn"] = rng.uniform(0.5, 1.5, (L, d)).astype(np.float32)
    m["rms_final"] = rng.uniform(0.5, 1.5, d).astype(np.float32)
    m["tok"][3, :] = 0.0  # a zero row: scale 1, all-zero codes
    return m


def expected(cfg, m):
    """The checker's quantization of the same f32 arrays."""
    want = {}
    for name in ("tok", "wq", "wk", "wv", "wo", "w1", "w2", "w3"):
        w = m[name]
        q, s = oracle.quantize_rows(w.reshape(-1, w.shape[-1]))
        key = "tok" if name == "tok" else name
        want[f"{key}_q"] = q.reshape(w.shape)
        want[f"{key}_s"] = s.reshape(w.shape[:-1])
    for name in ("rms_att", "rms_ffn", "rms_final"):
        want[name] = m[name]
    want["rope"] = llama.rope_table(cfg)
    return want


@pytest.mark.parametrize("rope_arrays", [True, False])
def test_checkpoint_quantized_like_the_checker(lib, tmp_path, rope_arrays):
    m = f32_model(CFG)
    path = tmp_path / "tiny.bin"
    write_checkpoint(path, CFG, m, rope_arrays=rope_arrays)
    cfg, got = read_model(lib, path)
    assert cfg == CFG
    want = expected(CFG, m)
    for name, arr in want.items():
        assert np.array_equal(got[name], arr), name
    assert not got["tok_q"][3].any() and got["tok_s"][3] == 1.0


def test_quantizer_agrees_with_numpy_restatement():
    """The checker's C quantizer against the numpy statement of the same rule
    (scale = max|w|/127, round half to even), including exact ties."""
    w = np.array([[127.0, 63.5, -0.5, 1.5, 2.5, -127.0]], np.float32)
    q, s = oracle.quantize_rows(w)
    assert s[0] == 1.0 and list(q[0]) == [127, 64, 0, 2, 2, -127]
    w = np.random.default_rng(0).standard_normal((64, 96)).astype(np.float32)
    q, s = oracle.quantize_rows(w)
    qn, sn = llama.quantize_rows(w)
    assert np.array_equal(q, qn) and np.array_equal(s, sn)


def test_q8_round_trip(lib, tmp_path):
    m = llama.make_model(CFG, seed=3)
    path = tmp_path / "tiny.q8"
    save_model(lib, path, CFG, m)
    cfg, got = read_model(lib, path)
    assert cfg == CFG
    for name in m:
        assert np.array_equal(got[name], m[name]), name
    # The file is the config plus every stored array, nothing else.
    stored = sum(a.nbytes for k, a in m.items() if k != "rope")
    assert path.stat().st_size == 8 + 28 + stored + 8


def test_checkpoint_then_q8_gives_the_same_model(lib, tmp_path):
    m = f32_model(CFG, seed=9)
    write_checkpoint(tmp_path / "a.bin", CFG, m)
    cfg, first = read_model(lib, tmp_path / "a.bin")
    save_model(lib, tmp_path / "a.q8", cfg, first)
    _, second = read_model(lib, tmp_path / "a.q8")
    for name in first:
        assert np.array_equal(first[name], second[name]), name


def test_refusals(lib, tmp_path):
    m = f32_model(CFG)
    good = tmp_path / "good.bin"
    write_checkpoint(good, CFG, m)
    data = good.read_bytes()
    with pytest.raises(OSError):
        read_model(lib, tmp_path / "missing.bin")
    (tmp_path / "short.bin").write_bytes(data[:-4])
    with pytest.raises(OSError):
        read_model(lib, tmp_path / "short.bin")
    neg = bytearray(data)
    neg[20:24] = np.int32(-CFG.vocab_size).tobytes()  # unshared classifier
    (tmp_path / "neg.bin").write_bytes(bytes(neg))
    with pytest.raises(OSError) as e:
        read_model(lib, tmp_path / "neg.bin")
    assert e.value.args[0] == -4  # VX_OP_EUNSUPP
    bad = bytearray(data)
    bad[12:16] = np.int32(5).tobytes()  # n_heads 5 does not divide dim 64
    (tmp_path / "bad.bin").write_bytes(bytes(bad))
    with pytest.raises(OSError):
        read_model(lib, tmp_path / "bad.bin")
    save_model(lib, tmp_path / "m.q8", CFG, llama.make_model(CFG))
    q8 = bytearray((tmp_path / "m.q8").read_bytes())
    q8[100] ^= 1
    (tmp_path / "flip.q8").write_bytes(bytes(q8))
    with pytest.raises(OSError):
        read_model(lib, tmp_path / "flip.q8")


def test_huge_vxq8_header_is_refused_before_allocating(lib, tmp_path):
    """A VXQ8 header that claims the largest config the reader accepts (dim
    2^16, hidden 2^18, 4096 layers, vocab 2^22) on a file of a few bytes is
    refused from the size check, without allocating the terabytes the
    header describes."""
    save_model(lib, tmp_path / "m.q8", CFG, llama.make_model(CFG))
    q8 = bytearray((tmp_path / "m.q8").read_bytes())
    q8[8:36] = np.array([1 << 16, 1 << 18, 4096, 1 << 10, 1 << 10, 1 << 22, 1 << 20],
                        dtype=np.int32).tobytes()
    (tmp_path / "huge.q8").write_bytes(bytes(q8))
    with pytest.raises(OSError) as e:
        read_model(lib, tmp_path / "huge.q8")
    assert e.value.args[0] == -1  # VX_OP_EINVAL: size disagrees with header


@pytest.mark.parametrize("cfg", [llama.CONFIG_TINY,
                                 llama.LlamaConfig(dim=96, hidden_dim=160, n_layers=3, n_heads=6,
                                                   n_kv_heads=2, vocab_size=300, seq_len=40)])
def test_step_byte_counts(cfg):
    """The bytes the decode roofline divides by: int8_weight_bytes() is every
    array of the uploaded model except the rotary table (int8 matrices, f32
    row scales, f32 RMSNorm weights), and kv_bytes(pos) is the f32 key and
    value rows 0..pos read plus row pos written, per layer, counted here
    element by element from the cache layout [layer][position][kv_dim]."""
    m = llama.make_model(cfg, seed=0)
    assert cfg.int8_weight_bytes() == sum(v.nbytes for k, v in m.items() if k != "rope")
    for pos in (0, 1, cfg.seq_len - 1):
        rows_read = pos + 1
        per_layer = 2 * (rows_read + 1) * cfg.kv_dim * np.dtype(np.float32).itemsize
        assert cfg.kv_bytes(pos) == cfg.n_layers * per_layer


# ---- the RoPE table against the reference's correctly rounded f32 maths ----

_DIGITS = 60


def _dec_pi():
    from decimal import Decimal
    return Decimal("3.14159265358979323846264338327950288419716939937510582097494459230781640628620899")


def _dec_cos_sin(x: float):
    """cos and sin of a double to about 55 digits: reduction by a 80-digit
    pi, then the Taylor series."""
    from decimal import Decimal, localcontext
    with localcontext() as ctx:
        ctx.prec = _DIGITS
        x = Decimal(x)
        two_pi = 2 * _dec_pi()
        r = x - (x / two_pi).to_integral_value() * two_pi
        eps = Decimal(10) ** -(_DIGITS - 5)
        out = []
        for first, start in ((Decimal(1), 0), (r, 1)):
            t, acc, i = first, Decimal(0), start
            while abs(t) > eps:
                acc += t
                i += 2
                t = -t * r * r / (i * (i - 1))
            out.append(acc)
        return out[0], out[1]


def _dec_pow10000(e: float):
    from decimal import Decimal, localcontext
    with localcontext() as ctx:
        ctx.prec = _DIGITS
        return (Decimal(e) * Decimal(10000).ln()).exp()


def _round_f32(d) -> np.float32:
    """The f32 nearest to the Decimal d (ties cannot occur at these digits)."""
    from decimal import Decimal
    f = np.float32(float(d))
    cands = [f, np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf))]
    return min(cands, key=lambda g: abs(Decimal(float(g)) - d))


def _near_midpoint(v: float, ulps: float = 64.0) -> bool:
    """Whether the double v lies within `ulps` double ulps of a point halfway
    between two f32 values (where a double evaluation off by under one ulp
    could round to the other f32)."""
    f = np.float32(v)
    up = np.nextafter(f, np.float32(np.inf)) if float(f) <= v else f
    lo = f if float(f) <= v else np.nextafter(f, np.float32(-np.inf))
    mid = (float(lo) + float(up)) / 2.0
    return abs(v - mid) <= ulps * abs(np.spacing(v))


@pytest.mark.parametrize("hs,positions", [(64, 1024), (128, 512), (16, 256)])
def test_rope_table_is_correctly_rounded(hs, positions):
    """Reference examples/llama.vx:244-246 takes f32 cos and sin of the f32
    angle pos * 10000^(-i/hs), with powf, cos and sin documented as correctly
    rounded (reference stdlib/core/num.vx:2434-2442, 2476-2479). Every
    inverse frequency is checked against a 60-digit power. Each table entry
    whose double evaluation lies near an f32 rounding midpoint (where a
    rounding of the double could differ from the correct one) is checked
    against a 60-digit cos/sin, and so are 200 entries picked at random; the
    others round correctly because glibc's double cos and sin are within one
    ulp. Config 4's table is the first case."""
    import math

    cfg = llama.LlamaConfig(dim=hs * 4, hidden_dim=64, n_layers=1, n_heads=4, n_kv_heads=4,
                            vocab_size=32, seq_len=positions)
    inv = llama.rope_inv_freq(hs)
    for j, i in enumerate(range(0, hs, 2)):
        e = float(-np.float32(i) / np.float32(hs))
        assert inv[j] == _round_f32(_dec_pow10000(e)), (hs, i)
    tab = llama.rope_table(cfg)
    assert tab.shape == (positions, hs // 2, 2)
    ang = (np.arange(positions, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    rng = np.random.default_rng(hs)
    sample = set(zip(rng.integers(0, positions, 200).tolist(), rng.integers(0, hs // 2, 200).tolist()))
    checked = 0
    for p in range(positions):
        for j in range(hs // 2):
            a = float(ang[p, j])
            if (p, j) in sample or _near_midpoint(math.cos(a)) or _near_midpoint(math.sin(a)):
                c, s = _dec_cos_sin(a)
                assert tab[p, j, 0] == _round_f32(c), (p, j, "cos")
                assert tab[p, j, 1] == _round_f32(s), (p, j, "sin")
                checked += 1
    assert checked >= len(sample)
