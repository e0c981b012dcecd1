"""GPU: fl_moe_layer_noalloc -- the allocation-free variant of fl_moe_layer for decode batches -- through the C ABI.

Its output must equal fl_moe_layer's bit for bit on the same inputs, on consecutive calls with shrinking batches (the
file-scope scratch keeps the previous call's contents), interleaved with the regular entry point, and with keep-2
routing; it must leave the context's own buffers unallocated and reject batches above its scratch's size. Captured
into a HIP graph, every replay on a new x must equal fl_moe_layer on that x."""
import ctypes

import numpy as np
import pytest

from tests._helpers import make_layer, make_x

pytestmark = pytest.mark.gpu


def _noalloc(ctx, layer, x, y):
    from loki_amd import lib
    return lib().fl_moe_layer_noalloc(ctx.ctx, ctypes.byref(layer.abi()), ctypes.c_void_p(x.data_ptr()), x.shape[0],
                                      ctypes.c_void_p(y.data_ptr()))


def test_noalloc_matches_moe_layer():
    import torch
    from loki_amd import FL_ERANGE, FL_OK, Context
    na = Context()    # a fresh context: the entry point must not allocate its buffers
    ref = Context()   # the regular entry point, on its own context
    try:
        layer = make_layer(ref, seed=4242)
        xs = {n: make_x(ref, n, seed=50 + n) for n in (8, 3, 1)}
        ys = {n: torch.empty_like(x) for n, x in xs.items()}
        # the HIP runtime loads a kernel's code object (and may size its private segment) at its first launch in the
        # process: launch every kernel once through the regular entry point before taking the baseline
        ref.moe_layer(layer, xs[8])
        ref.sync()
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        for n in (8, 3, 1):   # shrinking batches, back to back
            assert _noalloc(na, layer, xs[n], ys[n]) == FL_OK, n
        na.sync()
        free1 = torch.cuda.mem_get_info()[0]
        dbg = na.debug()
        assert not dbg.xq and not dbg.sel and not dbg.logits, "the context's buffers were allocated"
        assert free0 - free1 < (1 << 20), (free0, free1)
        for n in (8, 3, 1):
            want = ref.moe_layer(layer, xs[n]).cpu().numpy()
            assert np.array_equal(ys[n].cpu().numpy().view(np.uint32), want.view(np.uint32)), n
        # interleaved with the regular entry point, then again (epochs continue per device)
        y2 = torch.empty_like(xs[3])
        ref.moe_layer(layer, xs[8])
        assert _noalloc(na, layer, xs[3], y2) == FL_OK
        na.sync(); ref.sync()
        assert np.array_equal(y2.cpu().numpy().view(np.uint32), ys[3].cpu().numpy().view(np.uint32))
        # keep-2 routing (the reference engine's production setting) on both paths
        na.set_keep(2, 2.5); ref.set_keep(2, 2.5)
        y8 = torch.empty_like(xs[8])
        assert _noalloc(na, layer, xs[8], y8) == FL_OK
        na.sync()
        want = ref.moe_layer(layer, xs[8]).cpu().numpy()
        assert np.array_equal(y8.cpu().numpy().view(np.uint32), want.view(np.uint32))
        # a batch above the scratch's size is rejected before any launch
        x9 = make_x(ref, 9, seed=77)
        y9 = torch.empty_like(x9)
        assert _noalloc(na, layer, x9, y9) == FL_ERANGE
    finally:
        torch.cuda.synchronize()
        na.close(); ref.close()


@pytest.mark.parametrize("n", [1, 8])
def test_noalloc_graph_replays(n):
    """One call captured into a HIP graph (torch.cuda.CUDAGraph on the context's stream), replayed nine times over
    three inputs copied into the captured x, with the program's own eager work and a synchronisation between replays:
    every replay's y equals fl_moe_layer's on that input bit for bit (the one-token kernel at n = 1, the n <= 8 block at
    n = 8), and fl_sync reports no device error afterwards."""
    import torch
    from loki_amd import FL_OK, Context, lib
    na = Context()
    ref = Context()
    try:
        layer = make_layer(ref, seed=4243)
        xs = [make_x(ref, n, seed=300 + 10 * n + i) for i in range(3)]
        want = [ref.moe_layer(layer, x).cpu().numpy() for x in xs]
        ref.sync()
        x_in, y_out = torch.empty_like(xs[0]), torch.empty_like(xs[0])
        x_in.copy_(xs[0])
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        na.check(lib().fl_set_stream(na.ctx, ctypes.c_void_p(side.cuda_stream)))   # before the capture starts
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            rc = _noalloc(na, layer, x_in, y_out)
        na.check(lib().fl_set_stream(na.ctx, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
        assert rc == FL_OK
        for rep in range(3):
            for i, x in enumerate(xs):
                x_in.copy_(x)
                y_out.fill_(float("nan"))
                torch.cuda.synchronize()
                g.replay()
                torch.cuda.synchronize()
                got = y_out.cpu().numpy()
                assert np.array_equal(got.view(np.uint32), want[i].view(np.uint32)), (n, rep, i)
        na.sync()
        del g
    finally:
        torch.cuda.synchronize()
        na.close(); ref.close()
