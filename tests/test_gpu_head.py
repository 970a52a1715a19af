"""The LM head before the sampler (tc_lm_head, tc_head_sample) against an
exact product: the logits within the f32 accumulation's rounding bound of
float64 weight . hidden + bias, and the fused step's tokens equal to the
oracle sampling the device's own logits (the sampler is bit-exact given its
input; the head's summation order is this library's)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402
from talechime_amd import _lib, synth  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sampler():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from talechime_amd.sampler import DeviceSampler
    s = DeviceSampler(0, max_rows=64, max_vocab=1 << 14)
    yield s
    s.close()


def _case(rows, dim, vocab, wdt, bias, seed):
    g = np.random.default_rng(seed)
    h = g.standard_normal((rows, dim)).astype(np.float32)
    w = (g.standard_normal((vocab, dim)) * 0.05).astype(np.float32)
    if wdt == "bf16":
        wb = synth.to_bf16_bits(w)
        w = synth.bf16_bits_to_f32(wb)
        wt = torch.from_numpy(wb.view(np.int16)).view(torch.bfloat16).cuda()
    else:
        wt = torch.from_numpy(w).cuda()
    b = (g.standard_normal(vocab) * 0.5).astype(np.float32) if bias else None
    return h, w, b, wt


@pytest.mark.parametrize("rows,dim,vocab,wdt,bias", [
    (3, 1280, 8194, "bf16", True),     # indextts mel_head, one element x 3 beams (register kernel)
    (1, 1280, 8194, "f32", True),
    (2, 1280, 8194, "bf16", False),
    (4, 1024, 2048, "bf16", True),
    (16, 1024, 2048, "bf16", False),   # code predictor lm_head, 16 rows (two LDS chunks of 8)
    (5, 2048, 3072, "f32", False),
    (7, 4096, 1000, "bf16", True),     # chunks of 4 rows (8 do not fit the LDS)
    (61, 1280, 8194, "bf16", True),    # 8 chunks, the last partial
])
def test_lm_head_within_rounding_of_exact_product(sampler, rows, dim, vocab, wdt, bias):
    h, w, b, wt = _case(rows, dim, vocab, wdt, bias, rows * 1000 + dim)
    out = sampler.lm_head(torch.from_numpy(h).cuda(), wt, None if b is None else torch.from_numpy(b).cuda())
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    exact = h.astype(np.float64) @ w.astype(np.float64).T
    if b is not None:
        exact += b.astype(np.float64)
    # f32 accumulation over dim products: at most (dim + 8) roundings of the
    # running magnitudes, each 2^-24 of sum |w h|, plus the bias add
    mag = np.abs(h.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    bound = (dim + 8) * 2.0**-24 * mag + (0 if b is None else 2.0**-24 * (np.abs(exact) + 1e-30))
    err = np.abs(got - exact)
    print(f"[head] rows={rows} dim={dim} vocab={vocab} {wdt} max_err={err.max():.3e} "
          f"max_rel_to_bound={(err / bound).max():.3f}", flush=True)
    assert (err <= bound).all()


def test_head_sample_tokens_equal_oracle_on_device_logits(sampler):
    from talechime_amd.sampler import make_params
    rows, dim, vocab = 6, 1280, 8194
    h, w, b, wt = _case(rows, dim, vocab, "bf16", True, 7)
    w_ = synth.WORKLOADS["indextts-mel-256x8194"]
    bt = synth.make_batch(w_, rows=rows)
    kw = dict(temperature=0.8, top_k=30, top_p=0.8, penalty=10.0, min_keep=2)
    logits = torch.empty(rows, vocab, dtype=torch.float32, device="cuda")
    r = sampler.head_sample(make_params(_lib.INDEXTTS, **kw), torch.from_numpy(h).cuda(), wt,
                            torch.from_numpy(b).cuda(), torch.from_numpy(bt.hist_off.view(np.int32).copy()).cuda(),
                            torch.from_numpy(bt.hist_ids.view(np.int32).copy()).cuda(),
                            torch.from_numpy(bt.uniforms).cuda(), logits=logits)
    torch.cuda.synchronize()
    lg = logits.cpu().numpy()
    o = O.sample(O.make_params(O.INDEXTTS, **kw), lg, bt.hist_off, bt.hist_ids, bt.uniforms)
    assert (r.status.cpu().numpy() == 0).all()
    assert np.array_equal(r.ids.cpu().numpy().view(np.uint32), o["ids"])
    # and the qwen code-predictor shape: 2048-wide head without a bias
    rows, dim, vocab = 16, 1024, 2048
    h, w, _, wt = _case(rows, dim, vocab, "bf16", False, 8)
    u = np.random.default_rng(8).random(rows).astype(np.float32)
    logits = torch.empty(rows, vocab, dtype=torch.float32, device="cuda")
    r = sampler.head_sample(make_params(_lib.QWEN, temperature=0.9, top_k=50), torch.from_numpy(h).cuda(), wt,
                            None, None, None, torch.from_numpy(u).cuda(), logits=logits)
    torch.cuda.synchronize()
    o = O.sample(O.make_params(O.QWEN, temperature=0.9, top_k=50), logits.cpu().numpy(), None, None, u)
    assert np.array_equal(r.ids.cpu().numpy().view(np.uint32), o["ids"])


def test_lm_head_rejects_unsupported_shapes(sampler):
    wt = torch.zeros(16, 1283, dtype=torch.float32, device="cuda")
    with pytest.raises(_lib.TcError):
        sampler.lm_head(torch.zeros(1, 1283, device="cuda"), wt)
