"""GPU parity of the many-rows layer (d3_moe_a8_prefill: on-device grouping, grouped MFMA products) against the
oracle's layer (oracle/a8.py moe_layer), for all four A8 formats.

Bars as for the fused decode layer: routing ids exact and weights within one bf16 ulp; outputs (bf16) within max-abs
8e-3 * max|ref| (one bf16 step of any element) and rel-L2 3e-3 for
int8 / W4A8 / W6A8, 1.5e-2 and 6e-3 for FP8 (SiLU(gate) * up in float32 with a
fast exp before its quantization, the oracle in float64: a hidden code on a rounding boundary can differ by one step;
FP8 adds the MFMA's inner precision)."""
import numpy as np
import pytest
import torch

from drama3 import formats, moe
from oracle import a8
from oracle.numerics import bf16_bits_to_f32

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
FMTS = [formats.FMT_I8, formats.FMT_W4, formats.FMT_W6, formats.FMT_F8]
H, I = 2048, 768

_banks = {}


def banks(fmt, E=16, inter=I, seed=0):
    key = (fmt, E, inter, seed)
    if key not in _banks:
        _banks.clear()
        gen = torch.Generator(device=DEV).manual_seed(seed)
        gate_up = formats.quantize(torch.randn((E, 2 * inter, H), generator=gen, device=DEV) * 0.02, fmt)
        down = formats.quantize(torch.randn((E, H, inter), generator=gen, device=DEV) * 0.02, fmt)
        _banks[key] = (gate_up, down)
    return _banks[key]


def bits(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def fetcher(gate_up, down):
    cache = {}

    def fetch(bank, e):
        if (bank, e) not in cache:
            b = gate_up if bank == "gate_up" else down
            rows = slice(e * b.rows, (e + 1) * b.rows)
            cache[bank, e] = (b.weight[rows].cpu().numpy(),
                              b.scale[rows].contiguous().view(torch.int16).cpu().numpy().view(np.uint16))
        return cache[bank, e]
    return fetch


def check(fmt, x, logits, gate_up, down, topk=8):
    out, ids, w = moe.moe_prefill(x, gate_up, down, topk, logits=logits, routing=True)
    want, want_ids, want_w, _ = a8.moe_layer(bits(x), bits(logits), (gate_up.rows, gate_up.cols),
                                             (down.rows, down.cols), fmt, topk, fetcher(gate_up, down))
    assert np.array_equal(ids.cpu().numpy(), want_ids)
    assert np.all(np.abs(w.cpu().numpy() - want_w) <= np.abs(want_w) * 2.0 ** -8 + 1e-30)
    got = bf16_bits_to_f32(bits(out)).astype(np.float64)
    ref = bf16_bits_to_f32(want).astype(np.float64)
    assert np.all(np.isfinite(got))
    assert_layer_close(fmt, got, ref)
    return out, ids, w


def assert_layer_close(fmt, got, ref):
    max_bar, l2_bar = (1.5e-2, 6e-3) if fmt == formats.FMT_F8 else (8e-3, 3e-3)
    err = np.abs(got - ref)
    assert err.max() <= max_bar * np.abs(ref).max(), (err.max(), np.abs(ref).max())
    assert np.linalg.norm(got - ref) <= l2_bar * np.linalg.norm(ref), np.linalg.norm(got - ref) / np.linalg.norm(ref)


@pytest.mark.parametrize("fmt", FMTS)
def test_prefill_matches_oracle(fmt):
    gate_up, down = banks(fmt)
    gen = torch.Generator(device=DEV).manual_seed(20 + fmt)
    x = torch.randn((24, H), generator=gen, device=DEV).to(torch.bfloat16)
    logits = torch.randn((24, 16), generator=gen, device=DEV).to(torch.bfloat16)
    check(fmt, x, logits, gate_up, down)


@pytest.mark.parametrize("fmt", [formats.FMT_I8, formats.FMT_F8])
def test_prefill_hot_experts_many_tiles(fmt):
    """48 rows all routed to the same 8 experts: 48 pairs per expert, three 16-pair tiles each; 8 experts unused."""
    gate_up, down = banks(fmt)
    gen = torch.Generator(device=DEV).manual_seed(31)
    x = torch.randn((48, H), generator=gen, device=DEV).to(torch.bfloat16)
    logits = torch.randn((48, 16), generator=gen, device=DEV)
    logits[:, 3:11] += 20.0
    check(fmt, x, logits.to(torch.bfloat16), gate_up, down)


def test_prefill_single_row_and_reference_shape():
    """One row, and the reference model's shape (256 experts, FFN 512)."""
    gate_up, down = banks(formats.FMT_W4, E=256, inter=512, seed=5)
    gen = torch.Generator(device=DEV).manual_seed(32)
    for T in (1, 5):
        x = torch.randn((T, H), generator=gen, device=DEV).to(torch.bfloat16)
        logits = torch.randn((T, 256), generator=gen, device=DEV).to(torch.bfloat16)
        check(formats.FMT_W4, x, logits, gate_up, down)


@pytest.mark.parametrize("fmt", FMTS)
def test_few_rows_prep_in_one_launch(fmt):
    """Up to 16 rows route, quantize x and group in one launch; 17 rows take the wide launches (routing with x's
    quantization, then the grouping). Each output row depends on its own row only, so T rows and the first T of 17
    agree bit for bit; 1, 3, 7 and 16 rows match the oracle, with the routing given as well as computed."""
    gate_up, down = banks(fmt)
    gen = torch.Generator(device=DEV).manual_seed(40 + fmt)
    x = torch.randn((17, H), generator=gen, device=DEV).to(torch.bfloat16)
    logits = torch.randn((17, 16), generator=gen, device=DEV).to(torch.bfloat16)
    wide = moe.moe_prefill(x, gate_up, down, 8, logits=logits)
    for T in (1, 3, 7, 16):
        out, ids, w = check(fmt, x[:T].contiguous(), logits[:T].contiguous(), gate_up, down)
        assert torch.equal(out, wide[:T])
        assert torch.equal(moe.moe_prefill(x[:T].contiguous(), gate_up, down, 8, topk_idx=ids, topk_weight=w), out)


@pytest.mark.parametrize("fmt", [formats.FMT_I8, formats.FMT_W4])
@pytest.mark.parametrize("topk,T", [(2, 5), (2, 24), (16, 3), (16, 24), (12, 9)])
def test_prefill_other_topk(fmt, topk, T):
    """k other than 8: k 2 in the few-rows launch (5 rows) and the wide one; k 12 and 16 (every expert of 16) take
    the wide launches at any row count."""
    gate_up, down = banks(fmt)
    gen = torch.Generator(device=DEV).manual_seed(50 + topk + T)
    x = torch.randn((T, H), generator=gen, device=DEV).to(torch.bfloat16)
    logits = torch.randn((T, 16), generator=gen, device=DEV).to(torch.bfloat16)
    check(fmt, x, logits, gate_up, down, topk=topk)


@pytest.mark.parametrize("fmt", [formats.FMT_I8, formats.FMT_W6])
def test_given_routing_equals_logits_routing(fmt):
    """topk_idx / topk_weight handed in (as Experts.forward gets them) give the same output as routing inside."""
    gate_up, down = banks(fmt)
    gen = torch.Generator(device=DEV).manual_seed(33)
    x = torch.randn((20, H), generator=gen, device=DEV).to(torch.bfloat16)
    logits = torch.randn((20, 16), generator=gen, device=DEV).to(torch.bfloat16)
    out, ids, w = moe.moe_prefill(x, gate_up, down, 8, logits=logits, routing=True)
    again = moe.moe_prefill(x, gate_up, down, 8, topk_idx=ids, topk_weight=w)
    assert torch.equal(out, again)


@pytest.mark.parametrize("fmt", FMTS)
def test_prefill_close_to_fused_decode(fmt):
    """The same rows through the fused decode kernel and the prefill path: the same layer, other summation orders."""
    gate_up, down = banks(fmt)
    gen = torch.Generator(device=DEV).manual_seed(34)
    x = torch.randn((8, H), generator=gen, device=DEV).to(torch.bfloat16)
    logits = torch.randn((8, 16), generator=gen, device=DEV).to(torch.bfloat16)
    a = moe.moe_prefill(x, gate_up, down, 8, logits=logits).float()
    b = moe.moe_layer(x, logits, gate_up, down, 8, fused=True).float()
    assert torch.linalg.norm(a - b) <= 1e-2 * torch.linalg.norm(b)


@pytest.mark.parametrize("rows", [24, 16, 4])
def test_prefill_graph_replays(rows):
    gate_up, down = banks(formats.FMT_F8)
    gen = torch.Generator(device=DEV).manual_seed(35)
    xs = [torch.randn((rows, H), generator=gen, device=DEV).to(torch.bfloat16) for _ in range(3)]
    lgs = [torch.randn((rows, 16), generator=gen, device=DEV).to(torch.bfloat16) for _ in range(3)]
    x_buf, lg_buf = xs[0].clone(), lgs[0].clone()
    stream = torch.cuda.Stream(DEV)
    stream.wait_stream(torch.cuda.current_stream(DEV))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        moe.moe_prefill(x_buf, gate_up, down, 8, logits=lg_buf)
        with torch.cuda.graph(g, stream=stream):
            out = moe.moe_prefill(x_buf, gate_up, down, 8, logits=lg_buf)
    torch.cuda.current_stream(DEV).wait_stream(stream)
    for x, lg in zip(xs, lgs):
        x_buf.copy_(x)
        lg_buf.copy_(lg)
        g.replay()
        torch.cuda.synchronize()
        eager = moe.moe_prefill(x_buf, gate_up, down, 8, logits=lg_buf)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def zipf_logits(T, E, seed):
    """Router logits [T, E] bf16 drawn as bench.py draws the 256-row prefill's: log p(rank) with p(rank) ~ rank^-1.1
    over a seeded permutation of the experts, plus Gumbel noise, so each row's top-k is k distinct experts drawn from
    Zipf(1.1)."""
    gen = torch.Generator(device=DEV).manual_seed(seed)
    logp = -1.1 * torch.log(torch.arange(1, E + 1, device=DEV, dtype=torch.float32))
    perm = torch.randperm(E, generator=gen, device=DEV)
    base = torch.empty(E, device=DEV)
    base[perm] = logp
    u = torch.rand((T, E), generator=gen, device=DEV).clamp_(1e-12, 1 - 1e-7)
    return (base - torch.log(-torch.log(u))).to(torch.bfloat16)


def test_prefill_fp8_256_rows_zipf():
    """The prefill workload the benchmark times: 256 rows, FP8 experts at H 2048 / I 768, 128 experts, top-8 from
    Zipf(1.1)-skewed logits. The hottest expert holds more than 128 (row, expert) pairs, so it is split into work
    units of at most 128 pairs (the multi-unit path); every one of the 256 rows is checked against the oracle."""
    gate_up, down = banks(formats.FMT_F8, E=128, seed=7)
    gen = torch.Generator(device=DEV).manual_seed(70)
    x = torch.randn((256, H), generator=gen, device=DEV).to(torch.bfloat16)
    logits = zipf_logits(256, 128, seed=71)
    out, ids, w = check(formats.FMT_F8, x, logits, gate_up, down)
    counts = np.bincount(ids.cpu().numpy().ravel(), minlength=128)
    assert counts.max() > 128, counts.max()
    assert (counts > 0).sum() > 100  # most experts in use, as at this workload


@pytest.mark.parametrize("fmt,E,inter,T", [(formats.FMT_I8, 128, 768, 200), (formats.FMT_W4, 128, 768, 260),
                                           (formats.FMT_W6, 256, 512, 160)])
def test_prefill_experts_over_many_units(fmt, E, inter, T):
    """Rows biased onto a few experts: two experts take 150 to 260 pairs (2 or 3 work units of at most 128 pairs),
    the rest spread; against the oracle on every row."""
    gate_up, down = banks(fmt, E=E, inter=inter, seed=8)
    gen = torch.Generator(device=DEV).manual_seed(80 + fmt)
    x = torch.randn((T, H), generator=gen, device=DEV).to(torch.bfloat16)
    logits = torch.randn((T, E), generator=gen, device=DEV)
    logits[:, 5] += 20.0
    logits[: 150, E - 3] += 20.0
    out, ids, w = check(fmt, x, logits.to(torch.bfloat16), gate_up, down)
    counts = np.bincount(ids.cpu().numpy().ravel(), minlength=E)
    assert counts[5] == T and counts[E - 3] >= 150


@pytest.mark.parametrize("fmt", [formats.FMT_F8, formats.FMT_I8])
def test_prefill_rows_independent_at_1024_rows(fmt):
    """A size-independent check past the oracle's sizes: each output row depends only on its own row (its routing,
    its pairs' hidden rows quantized per pair, each MFMA column its own dot products, its k partial outputs summed in
    routing order), so 1024 rows at once (experts of up to ~900 pairs, split into many work units) equal, bit for
    bit, the same rows run 16 at a time (the one-launch prep) and one at a time."""
    gate_up, down = banks(fmt, E=128, seed=11)
    gen = torch.Generator(device=DEV).manual_seed(110 + fmt)
    T = 1024
    x = torch.randn((T, H), generator=gen, device=DEV).to(torch.bfloat16)
    logits = zipf_logits(T, 128, seed=111 + fmt)
    out, ids, w = moe.moe_prefill(x, gate_up, down, 8, logits=logits, routing=True)
    counts = np.bincount(ids.cpu().numpy().ravel(), minlength=128)
    assert counts.max() > 4 * 128  # the hottest expert spans five or more work units
    hot = int(np.argmax(counts))
    hot_rows = torch.nonzero((ids == hot).any(dim=1)).flatten()[:16]
    pick = torch.randperm(T, generator=torch.Generator().manual_seed(5))[:16].to(DEV)
    for rows in (torch.arange(16, device=DEV), pick, hot_rows):
        part, pids, pw = moe.moe_prefill(x[rows].contiguous(), gate_up, down, 8, logits=logits[rows].contiguous(),
                                         routing=True)
        assert torch.equal(pids, ids[rows]) and torch.equal(pw, w[rows])
        assert torch.equal(part, out[rows])
    for r in (0, int(hot_rows[0])):
        one = moe.moe_prefill(x[r:r + 1], gate_up, down, 8, logits=logits[r:r + 1])
        assert torch.equal(one, out[r:r + 1])
