"""GPU parity of the LM head with the int8 pre-pass (fw_lm_head_argmax_q8) against the fp16 LM head
(fw_lm_head_argmax_fused) and the CPU oracle. The packed winner (fp16 logit bits and index) must be
identical, bit for bit, on the seeded 51866 x 1280 table and on tables built to stress the pre-pass:
exact ties, near-ties below one fp16 ulp, all-equal logits (y = 0), logits that overflow fp16, heavy
suppression and odd vocabulary sizes. The int8 table's stored error bounds must bound the true
quantization error."""

import numpy as np
import pytest
import torch

from oracle import decoder as odec
from test_gpu_decode import h16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def ext(hip_device):
    from flash_whisper_amd.ext import load_ext

    return load_ext()


@pytest.fixture(scope='module')
def table(hip_device, ext):
    from flash_whisper_amd import weights

    w = torch.empty(51866, 1280, dtype=torch.float16, device=hip_device)
    weights.device_fill(w, 'model.decoder.embed_tokens.weight', 'normal', seed=0)
    wq, meta = ext.lm_head_q8_table(w)
    return w, wq, meta


def _best(ext, dev, q8, h, x, g, b, w, wq, meta, sup):
    best = torch.zeros(1, dtype=torch.long, device=dev)
    if q8:
        ext.lm_head_argmax_q8(h, x, g, b, 1e-5, w, wq, meta, sup, best, None, None, None, 448)
    else:
        ext.lm_head_argmax_fused(h, x, g, b, 1e-5, w, sup, best, None, None, None, 448)
    return int(best)


def _both(ext, dev, w, wq, meta, sup, h, x=None, g=None, b=None):
    g = torch.ones(1280, dtype=torch.float16, device=dev) if g is None else g
    b = torch.zeros(1280, dtype=torch.float16, device=dev) if b is None else b
    ref = _best(ext, dev, False, h, x, g, b, w, wq, meta, sup)
    got = _best(ext, dev, True, h, x, g, b, w, wq, meta, sup)
    return got, ref


def _token(packed):
    return 0xFFFFFFFF - (packed & 0xFFFFFFFF)


def test_q8_pack_error_bounds(ext, hip_device, table):
    w, wq, meta = table
    rows = np.random.default_rng(0).choice(w.size(0), 3000, replace=False)
    e = w[rows].double().cpu().numpy()
    q = wq[rows].cpu().numpy().astype(np.float64)
    m = meta[rows].cpu().numpy().astype(np.float64)
    assert np.abs(q).max() <= 127
    amax = np.abs(e).max(1)
    assert np.allclose(m[:, 0], amax / 127, rtol=2 ** -22, atol=0)
    err = np.sqrt(((e - m[:, :1] * q) ** 2).sum(1))
    assert (m[:, 1] >= err).all() and (m[:, 1] <= err * (1 + 1e-6) + 1e-30).all()
    assert np.abs(q - e / m[:, :1]).max() <= 0.5 + 1e-3  # nearest level


def test_q8_matches_fp16_head_on_seeded_table(ext, hip_device, table):
    from flash_whisper_amd import weights

    dev = hip_device
    w, wq, meta = table
    rng = np.random.default_rng(11)
    sup = torch.zeros(51866, dtype=torch.bool, device=dev)
    sup[torch.from_numpy(rng.choice(51866, 90, replace=False)).to(dev)] = True
    for trial in range(8):
        h = h16(rng.standard_normal(1280) * (1 + 3 * trial), dev)
        x = h16(rng.standard_normal(1280), dev) if trial % 2 else None
        g = h16(1 + 0.3 * rng.standard_normal(1280), dev) if trial >= 4 else None
        b = h16(0.2 * rng.standard_normal(1280), dev) if trial >= 4 else None
        got, ref = _both(ext, dev, w, wq, meta, sup, h, x, g, b)
        assert got == ref != 0, (trial, hex(got), hex(ref))
    # and the oracle's token on the seeded table (fp16 logits, lowest index on ties)
    w_np = weights.host_normal('model.decoder.embed_tokens.weight', (51866, 1280), seed=0)
    hn = np.float16(rng.standard_normal(1280))
    g1, b0 = np.ones(1280, np.float16), np.zeros(1280, np.float16)
    _, y = odec.add_layernorm(hn, None, g1, b0, 1e-5)
    tok = odec.lm_head_argmax(y, w_np, sup.cpu().numpy())
    got, ref = _both(ext, dev, w, wq, meta, sup, h16(hn, dev))
    assert got == ref and _token(got) == tok


def test_q8_finalize_steps(ext, hip_device, table):
    """Three fused steps in a row, as inside the decoder graph: each appends the token and leaves best 0."""
    dev = hip_device
    w, wq, meta = table
    rng = np.random.default_rng(3)
    h = h16(rng.standard_normal(1280), dev)
    g, b = torch.ones(1280, dtype=torch.float16, device=dev), torch.zeros(1280, dtype=torch.float16, device=dev)
    sup = torch.zeros(51866, dtype=torch.bool, device=dev)
    ref = _token(_best(ext, dev, False, h, None, g, b, w, wq, meta, sup))
    best = torch.zeros(1, dtype=torch.long, device=dev)
    tokens, state = torch.zeros(448, dtype=torch.long, device=dev), torch.tensor([3, 0], device=dev)
    cur = torch.zeros(1, dtype=torch.long, device=dev)
    for i in range(3):
        ext.lm_head_argmax_q8(h, None, g, b, 1e-5, w, wq, meta, sup, best, tokens, state, cur, 448)
        assert tokens[:i + 1].tolist() == [ref] * (i + 1) and state.tolist() == [4 + i, 1 + i]
        assert int(cur) == ref and int(best) == 0


def _small_case(dev, ext, w_np, sup_idx=(), y=None, gamma=None, beta=None):
    vocab = w_np.shape[0]
    tw = h16(w_np, dev)
    wq, meta = ext.lm_head_q8_table(tw)
    sup = torch.zeros(vocab, dtype=torch.bool, device=dev)
    if len(sup_idx):
        sup[list(sup_idx)] = True
    rng = np.random.default_rng(vocab)
    h = h16(rng.standard_normal(1280) if y is None else y, dev)
    g = None if gamma is None else h16(gamma, dev)
    b = None if beta is None else h16(beta, dev)
    return _both(ext, dev, tw, wq, meta, sup, h, None, g, b)


def test_q8_exact_ties_and_suppression(ext, hip_device):
    dev = hip_device
    rng = np.random.default_rng(5)
    w = np.float16(0.02 * rng.standard_normal((4099, 1280)))
    y = rng.standard_normal(1280)
    w[[100, 2000, 4098]] = np.float16(0.05 * np.sign(y))  # identical clear winners
    for sup_idx, expect in (((), 100), ((100,), 2000), ((100, 2000), 4098)):
        got, ref = _small_case(dev, ext, w, sup_idx, y=y)
        assert got == ref and _token(got) == expect


def test_q8_near_ties(ext, hip_device):
    """Rows that differ from one row in a few elements by one fp16 ulp: their logits agree to far below
    the pre-pass bound, so the exact pass decides among many candidates."""
    dev = hip_device
    rng = np.random.default_rng(8)
    w = np.float16(0.02 * rng.standard_normal((8192, 1280)))
    base = np.float16(0.03 * rng.standard_normal(1280))
    for k in range(3000, 3400):
        r = base.copy()
        idx = rng.choice(1280, 3, replace=False)
        r[idx] = np.nextafter(r[idx], np.float16(np.inf) if k % 2 else np.float16(-np.inf))
        w[k] = r
    y = np.float16(np.sign(base.astype(np.float32)) * np.abs(rng.standard_normal(1280)))
    for sup_idx in ((), tuple(range(3000, 3400, 3))):
        got, ref = _small_case(dev, ext, w, sup_idx, y=y)
        assert got == ref != 0


def test_q8_all_equal_and_overflowing_logits(ext, hip_device):
    dev = hip_device
    rng = np.random.default_rng(9)
    w = np.float16(0.02 * rng.standard_normal((3000, 1280)))
    zeros = np.zeros(1280)
    # y = 0 (gamma = beta = 0): every logit is 0, the lowest unsuppressed index wins
    got, ref = _small_case(dev, ext, w, (0, 1, 5), gamma=zeros, beta=zeros)
    assert got == ref and _token(got) == 2
    # y = 60000 everywhere: logits of rows with a positive sum overflow to +inf and tie there
    w2 = w.copy()
    w2[[700, 1200]] = np.float16(0.01)
    got, ref = _small_case(dev, ext, w2, (), gamma=zeros, beta=np.full(1280, 60000.0))
    assert got == ref != 0
    # all logits overflow to -inf: the lowest unsuppressed index wins
    w3 = np.float16(np.full((600, 1280), -0.01))
    got, ref = _small_case(dev, ext, w3, (0,), gamma=zeros, beta=np.full(1280, 60000.0))
    assert got == ref and _token(got) == 1


@pytest.mark.parametrize('vocab', [1, 63, 64, 65, 257, 1000, 16411])
def test_q8_odd_vocab_sizes(ext, hip_device, vocab):
    dev = hip_device
    rng = np.random.default_rng(vocab + 1)
    w = np.float16(0.02 * rng.standard_normal((vocab, 1280)))
    w[rng.integers(vocab)] = 0  # an all-zero row (scale 0)
    got, ref = _small_case(dev, ext, w, ())
    assert got == ref != 0


def test_q8_argument_checks(ext, hip_device, table):
    dev = hip_device
    w, wq, meta = table
    g, b = torch.ones(1280, dtype=torch.float16, device=dev), torch.zeros(1280, dtype=torch.float16, device=dev)
    h = torch.zeros(1280, dtype=torch.float16, device=dev)
    sup = torch.zeros(51866, dtype=torch.bool, device=dev)
    best = torch.zeros(1, dtype=torch.long, device=dev)
    with pytest.raises(RuntimeError, match='wq must match w'):
        ext.lm_head_argmax_q8(h, None, g, b, 1e-5, w, wq[:100], meta, sup, best, None, None, None, 448)
    with pytest.raises(RuntimeError, match='given together'):
        ext.lm_head_argmax_q8(h, None, g, b, 1e-5, w, wq, meta, sup, best, best, None, None, 448)
    with pytest.raises(RuntimeError, match='int8'):
        ext.lm_head_argmax_q8(h, None, g, b, 1e-5, w, wq.view(torch.uint8), meta, sup, best, None, None, None, 448)
