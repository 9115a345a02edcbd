"""The entry point that allocates nothing (d3_moe_a8_noalloc): the fused layer with its workspace in a static device
array of the library, against d3_moe_a8 with a workspace the caller allocated, bit for bit, on two calls in a row
(the second a smaller layer), its refusal of a layer larger than the static workspace, the call captured in a graph
and replayed, and its status reader."""
import ctypes

import pytest
import torch

from drama3 import _lib, formats, moe

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _noalloc():
    return _lib.lib().d3_moe_a8_noalloc


def _banks(fmt, E, I, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    gate_up = formats.quantize(torch.randn((E, 2 * I, 2048), generator=gen, device=DEV) * 0.02, fmt)
    down = formats.quantize(torch.randn((E, 2048, I), generator=gen, device=DEV) * 0.02, fmt)
    return gate_up, down


def _call(fn, x, logits, gate_up, down, topk, I, E):
    M = x.shape[0]
    out = torch.empty((M, 2048), dtype=torch.bfloat16, device=DEV)
    ids = torch.empty((M, topk), dtype=torch.int64, device=DEV)
    weights = torch.empty((M, topk), dtype=torch.float32, device=DEV)
    desc = _lib.MoeA8Desc(
        x=x.data_ptr(), logits=logits.data_ptr(), gate_up=gate_up.weight.data_ptr(),
        gate_up_scale=gate_up.scale.data_ptr(), down=down.weight.data_ptr(), down_scale=down.scale.data_ptr(),
        out=out.data_ptr(), ids_out=ids.data_ptr(), weights_out=weights.data_ptr(), workspace=None,
        workspace_bytes=0, format=gate_up.fmt, M=M, H=2048, I=I, E=E, topk=topk)
    rc = fn(ctypes.byref(desc), _lib.stream_of(DEV))
    return rc, out, ids, weights


def test_noalloc_matches_the_allocating_entry():
    fn = _noalloc()
    cases = [(formats.FMT_W4, 4, 768, 128, 1), (formats.FMT_I8, 1, 512, 256, 2)]  # the second call: a smaller layer
    for fmt, M, I, E, seed in cases:
        gate_up, down = _banks(fmt, E, I, seed)
        gen = torch.Generator(device=DEV).manual_seed(10 + seed)
        x = torch.randn((M, 2048), generator=gen, device=DEV).to(torch.bfloat16)
        logits = torch.randn((M, E), generator=gen, device=DEV).to(torch.bfloat16)
        want, want_ids, want_w = moe.moe_layer(x, logits, gate_up, down, 8, routing=True, fused=True)
        rc, out, ids, weights = _call(fn, x, logits, gate_up, down, 8, I, E)
        _lib.check(rc, "d3_moe_a8_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        assert torch.equal(ids, want_ids) and torch.equal(weights, want_w)


def test_noalloc_rejects_layers_beyond_its_workspace():
    fn = _noalloc()
    gate_up, down = _banks(formats.FMT_I8, 8, 512, 3)
    x = torch.zeros((16, 2048), dtype=torch.bfloat16, device=DEV)
    logits = torch.zeros((16, 8), dtype=torch.bfloat16, device=DEV)
    # 16 rows at I 1024: more workspace than the static array holds (refused before any launch)
    rc, *_ = _call(fn, x, logits, gate_up, down, 8, 1024, 8)
    assert rc != 0
    assert "static one" in _lib.lib().d3_last_error().decode()


def test_noalloc_captured_in_a_graph_and_replayed():
    """The call recorded into a graph (the first noalloc call of the process when this test runs alone) and replayed
    four times, with eager work and synchronizations between the replays: every replay equals the allocating entry's
    output bit for bit, and the noalloc status reads no failed wait."""
    fn = _lib.lib().d3_moe_a8_noalloc
    E, I, M = 128, 768, 1
    gate_up, down = _banks(formats.FMT_I8, E, I, 21)
    gen = torch.Generator(device=DEV).manual_seed(22)
    xs = [torch.randn((M, 2048), generator=gen, device=DEV).to(torch.bfloat16) for _ in range(4)]
    logits = [torch.randn((M, E), generator=gen, device=DEV).to(torch.bfloat16) for _ in range(4)]
    wants = [moe.moe_layer(x, lg, gate_up, down, 8, fused=True) for x, lg in zip(xs, logits)]
    x_buf, lg_buf = xs[0].clone(), logits[0].clone()
    out = torch.empty((M, 2048), dtype=torch.bfloat16, device=DEV)
    desc = _lib.MoeA8Desc(
        x=x_buf.data_ptr(), logits=lg_buf.data_ptr(), gate_up=gate_up.weight.data_ptr(),
        gate_up_scale=gate_up.scale.data_ptr(), down=down.weight.data_ptr(), down_scale=down.scale.data_ptr(),
        out=out.data_ptr(), ids_out=None, weights_out=None, workspace=None, workspace_bytes=0, format=gate_up.fmt,
        M=M, H=2048, I=I, E=E, topk=8)
    stream = torch.cuda.Stream(DEV)
    stream.wait_stream(torch.cuda.current_stream(DEV))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            _lib.check(fn(ctypes.byref(desc), ctypes.c_void_p(stream.cuda_stream)), "d3_moe_a8_noalloc")
    torch.cuda.synchronize()
    for i in range(4):
        x_buf.copy_(xs[i])
        lg_buf.copy_(logits[i])
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, wants[i]), i
        scratch = torch.randn((1 << 16,), device=DEV).sum()   # eager work between the replays
        torch.cuda.synchronize()
        del scratch
    status = ctypes.c_uint32(0xFFFFFFFF)
    _lib.check(_lib.lib().d3_moe_a8_noalloc_status(ctypes.byref(status)), "d3_moe_a8_noalloc_status")
    assert status.value & moe.STATUS_INVALID == 0
    again = ctypes.c_uint32(0xFFFFFFFF)
    _lib.check(_lib.lib().d3_moe_a8_noalloc_status(ctypes.byref(again)), "d3_moe_a8_noalloc_status")
    assert again.value == 0   # read and cleared
