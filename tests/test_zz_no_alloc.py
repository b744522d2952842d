"""GPU parity: pkv_attn_decode_step_noalloc (the fused decode step with the
library's per-GPU device array as workspace) against pkv_attn_decode_step
with a caller workspace, on two calls in a row (the second smaller, so it
runs over what the first left in the array): outputs and caches bit-equal,
outputs within the north-star tolerance of the oracle (max-abs 2e-3,
rel 1e-2)."""
import numpy as np
import pytest
import torch

import pkv
from _util import BS, D, close
from test_gpu_step import SCALE, i16, i32, oracle_step, step_case

pytestmark = pytest.mark.gpu


def run_step(c, dev, noalloc):
    Hq, Hkv, T = c["Hq"], c["Hkv"], c["T"]
    kc, vc = i16(c["kc"], dev), i16(c["vc"], dev)
    q, qkv = i16(c["q"], dev), i16(c["qkv"], dev)
    pos, ts, bt, cu, slot = (i32(c[k], dev) for k in ("pos", "tok_seq", "bt", "cu", "slot"))
    outs = i32(c["outs"], dev)
    out = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev)
    k_rows = qkv.data_ptr() + 2 * (2 * Hq * D)
    v_rows = k_rows + 2 * Hkv * D
    args = (k_rows, v_rows, c["qstride"] * 2, slot, q, kc, vc, qkv, c["qstride"], Hq, Hkv, pos, ts, bt,
            c["max_blocks"], BS, out, SCALE, cu, 0, outs, 1, T, c["pages"])
    if noalloc:
        pkv.attn_decode_step_noalloc(*args)
    else:
        ws = torch.empty(pkv.attn_decode_workspace(T, Hq), dtype=torch.uint8, device=dev)
        pkv.attn_decode_step(*args, ws)
    torch.cuda.synchronize()
    return (out.cpu().numpy().view(np.uint16), kc.cpu().numpy().view(np.uint16), vc.cpu().numpy().view(np.uint16))


def test_noalloc_step_matches_workspace_step_twice(dev):
    pkv.attn_decode_config(1, 32)
    rng = np.random.default_rng(7)
    big = [int(x) for x in rng.integers(512, 8193, 64)]   # C3-shaped: 64 sequences, 512..8192 keys
    small = [int(x) for x in rng.integers(1, 600, 5)]     # fewer tokens: reuses the array's leftovers
    for i, (lens, Hkv, per_seq) in enumerate([(big, 4, 1), (small, 4, 2)]):
        print(f"case noalloc call {i} B={len(lens)} Hkv={Hkv} per_seq={per_seq}", flush=True)
        c = step_case(lens, Hkv, 40 + i, per_seq)
        n_out, n_kc, n_vc = run_step(c, dev, noalloc=True)
        w_out, w_kc, w_vc = run_step(c, dev, noalloc=False)
        assert np.array_equal(n_out, w_out), f"call {i}: outputs differ from pkv_attn_decode_step"
        assert np.array_equal(n_kc, w_kc) and np.array_equal(n_vc, w_vc), f"call {i}: caches differ"
        o_out, o_kc, o_vc = oracle_step(c)
        assert np.array_equal(n_kc, o_kc) and np.array_equal(n_vc, o_vc), f"call {i}: append differs from oracle"
        ok, err = close(n_out, o_out)
        assert ok, f"call {i}: max |diff| {err}"


def test_noalloc_step_rejects_a_step_beyond_the_array(dev):
    L = pkv._lib
    # T = 4096 tokens at Hq = 16 needs ~70 MiB of partials: refused before any launch
    st = L.pkv_attn_decode_step_noalloc(16, 16, 10240 * 2, 16, 16, 16, 16, 16, 10240, 16, 4, 16, 16, 16, 4, 16, 16,
                                        0.1, 16, 0, None, 1, 4096, 10, None)
    assert st == pkv.ERR_UNSUPPORTED
