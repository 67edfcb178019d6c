"""The no-allocation layer decode (cachalot_moe_layer_decode_q2_static) against
the workspace entry point (cachalot_moe_layer_decode_q2), through the C ABI:
ids, weights, scores, routed and out bit for bit, on calls in a row of
decreasing size (the static scratch keeps the previous call's contents), and
the size check."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import SEED, make_store

pytestmark = pytest.mark.gpu


def _call(L, which, x, w, b, store, layer, k, addend):
    from cachalot_amd import _lib

    fmt = store.pool.format
    D, F = fmt.d_model, fmt.d_ff
    E = w.shape[0]
    dev = x.device
    idx = torch.full((k,), -7, dtype=torch.int32, device=dev)
    wt = torch.full((k,), -7.0, dtype=torch.float32, device=dev)
    scores = torch.full((E,), -7.0, dtype=torch.float32, device=dev)
    routed = torch.full((D,), -7.0, dtype=torch.float32, device=dev)
    out = torch.zeros((D,), dtype=torch.bfloat16, device=dev)
    table = store.layer_table(layer)
    head = (x.data_ptr(), w.data_ptr(), b.data_ptr(), E, k, _lib.SCORE_SIGMOID, 1.0, 1.0, 1, _lib.ORDER_ASCENDING,
            store.pool.storage.data_ptr(), store.pool.layout(), table.data_ptr(), D, F, 128, 10.0,
            addend.data_ptr(), idx.data_ptr(), wt.data_ptr(), scores.data_ptr(), routed.data_ptr(), out.data_ptr())
    stream = _lib.stream_handle(dev)
    if which == "static":
        rc = L.cachalot_moe_layer_decode_q2_static(*head, stream)
    else:
        nbytes = L.cachalot_moe_decode_q2_workspace_bytes(D, F, k)
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        rc = L.cachalot_moe_layer_decode_q2(*head, ws.data_ptr(), nbytes, stream)
    _lib.check(rc, which)
    torch.cuda.synchronize()
    return [t.cpu() for t in (idx, wt, scores, routed, out)]


def test_static_decode_matches_workspace_entry_point(cuda):
    from cachalot_amd import _lib, synth
    from cachalot_amd.storage.index import affine_format

    L = _lib.lib()
    cases = [(4096, 2880, 384, 6), (1024, 512, 64, 4), (4096, 2880, 384, 6)]   # big, smaller, big again
    stores = {}
    for n, (D, F, E, k) in enumerate(cases):
        print(f"no-alloc case {n}: D={D} F={F} E={E} k={k}", flush=True)
        if (D, F) not in stores:
            stores[(D, F)] = make_store(affine_format(D, F), n_layers=1, n_experts=E)
        store = stores[(D, F)]
        w, b = synth.router_weights(SEED, 0, E, D, cuda)
        x = synth.activations(SEED, 500 + n, 1, D, cuda)[0]
        a = synth.activations(SEED, 600 + n, 1, D, cuda)[0]
        want = _call(L, "workspace", x, w, b, store, 0, k, a)
        got = _call(L, "static", x, w, b, store, 0, k, a)
        for name, g, v in zip(("ids", "weights", "scores", "routed", "out"), got, want):
            assert torch.equal(g.view(torch.int32) if g.dtype == torch.float32 else g,
                               v.view(torch.int32) if v.dtype == torch.float32 else v), (n, name)
        assert int((got[0] >= 0).sum()) == k and np.isfinite(got[3].numpy()).all()


def test_static_decode_rejects_oversized_shapes(cuda):
    from cachalot_amd import _lib

    L = _lib.lib()
    limit = L.cachalot_moe_layer_decode_q2_static_max_bytes()
    assert L.cachalot_moe_decode_q2_workspace_bytes(8192, 8192, 8) > limit
    rc = L.cachalot_moe_layer_decode_q2_static(None, None, None, 384, 8, 1, 1.0, 1.0, 1, 0, None, None, None, 8192,
                                               8192, 128, 10.0, None, None, None, None, None, None,
                                               _lib.stream_handle(cuda))
    assert rc == _lib.ESPACE and "static array holds" in _lib.last_error()
