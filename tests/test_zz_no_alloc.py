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


def test_noalloc_step_g6_matches_workspace_step_twice(dev):
    """The reference's 27B shape (24 query heads over 4 kv heads: the verify
    kernel's records, 2 per index) at C3's batch: the no-allocation step
    equals the workspace step bit for bit on two calls in a row, the second
    smaller, and is within tolerance of the oracle."""
    pkv.attn_decode_config(1, 32)
    rng = np.random.default_rng(17)
    big = [int(x) for x in rng.integers(512, 8193, 64)]
    small = [int(x) for x in rng.integers(1, 900, 7)]
    for i, (lens, per_seq) in enumerate([(big, 1), (small, 2)]):
        print(f"case noalloc G=6 call {i} B={len(lens)} per_seq={per_seq}", flush=True)
        c = step_case(lens, 4, 60 + i, per_seq, G=6)
        n_out, n_kc, n_vc = run_step(c, dev, noalloc=True)
        w_out, w_kc, w_vc = run_step(c, dev, noalloc=False)
        assert np.array_equal(n_out, w_out), f"call {i}: outputs differ from pkv_attn_decode_step"
        assert np.array_equal(n_kc, w_kc) and np.array_equal(n_vc, w_vc), f"call {i}: caches differ"
        o_out, o_kc, o_vc = oracle_step(c)
        assert np.array_equal(n_kc, o_kc) and np.array_equal(n_vc, o_vc), f"call {i}: append differs from oracle"
        ok, err = close(n_out, o_out, what=f"noalloc G=6 call {i}")
        assert ok, f"call {i}: max |diff| {err}"


def test_noalloc_step_rejects_a_step_beyond_the_array(dev):
    L = pkv._lib
    # T = 4096 tokens at Hq = 16 needs ~70 MiB of partials: refused before any launch
    st = L.pkv_attn_decode_step_noalloc(16, 16, 10240 * 2, 16, 16, 16, 16, 16, 10240, 16, 4, 16, 16, 16, 4, 16, 16,
                                        0.1, 16, 0, None, 1, 4096, 10, None)
    assert st == pkv.ERR_UNSUPPORTED


_CAPTURE_CHILD = r'''
import sys
sys.path[:0] = [{root!r}, {root!r} + "/pocket-engine_amd", {root!r} + "/tests"]
import numpy as np, torch
import pkv
from _util import BS, D
from test_gpu_step import SCALE, i16, i32, step_case
dev = torch.device("cuda:0")
pkv.attn_decode_config(1, 32)
c = step_case([3000, 700, 41, 5000, 260], 4, 77, 1)
Hq, Hkv, T = c["Hq"], c["Hkv"], c["T"]
kc, vc = i16(c["kc"], dev), i16(c["vc"], dev)
q, qkv = i16(c["q"], dev), i16(c["qkv"], dev)
pos, ts, bt, cu, slot = (i32(c[k], dev) for k in ("pos", "tok_seq", "bt", "cu", "slot"))
out = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev)
k_rows = qkv.data_ptr() + 2 * (2 * Hq * D)
args = lambda o: (k_rows, k_rows + 2 * Hkv * D, c["qstride"] * 2, slot, q, kc, vc, qkv, c["qstride"], Hq, Hkv, pos,
                  ts, bt, c["max_blocks"], BS, o, SCALE, cu, 0, None, 1, T, c["pages"])
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    pkv.attn_decode_step_noalloc(*args(out))  # the process's first no-allocation call: inside the capture
ref = torch.zeros_like(out)
ws = torch.empty(pkv.attn_decode_workspace(T, Hq), dtype=torch.uint8, device=dev)
for r in range(3):
    out.fill_(0)
    g.replay()
    torch.cuda.synchronize()
    pkv.attn_decode_step(*args(ref), ws)  # eager work between replays
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"replay {{r}} differs from the workspace step"
print("capture ok", flush=True)
'''


def test_noalloc_first_call_inside_graph_capture(dev):
    """The first no-allocation call of a process (scratch address not yet
    looked up) made under HIP graph capture: the captured step replays three
    times, with eager workspace steps in between, each equal to them bit for
    bit. Runs in a child process so the lookup has not happened yet."""
    import os
    import subprocess
    import sys
    print("case noalloc first call under capture (child process)", flush=True)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD.format(root=root)], capture_output=True, text=True,
                       timeout=110)
    assert r.returncode == 0 and "capture ok" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]


def test_noalloc_step_allocates_no_device_memory(dev):
    """After a warm-up call, device free memory (hipMemGetInfo) is the same
    before and after several no-allocation steps."""
    import ctypes
    print("case noalloc free memory unchanged", flush=True)
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]

    def free_bytes():
        torch.cuda.synchronize()
        f, t = ctypes.c_size_t(), ctypes.c_size_t()
        assert hip.hipMemGetInfo(ctypes.byref(f), ctypes.byref(t)) == 0
        return f.value

    pkv.attn_decode_config(1, 32)
    c = step_case([2000, 90, 4100], 4, 78, 1)
    Hq, Hkv, T = c["Hq"], c["Hkv"], c["T"]
    kc, vc = i16(c["kc"], dev), i16(c["vc"], dev)
    q, qkv = i16(c["q"], dev), i16(c["qkv"], dev)
    pos, ts, bt, cu, slot = (i32(c[k], dev) for k in ("pos", "tok_seq", "bt", "cu", "slot"))
    out = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev)
    k_rows = qkv.data_ptr() + 2 * (2 * Hq * D)
    args = (k_rows, k_rows + 2 * Hkv * D, c["qstride"] * 2, slot, q, kc, vc, qkv, c["qstride"], Hq, Hkv, pos, ts, bt,
            c["max_blocks"], BS, out, SCALE, cu, 0, None, 1, T, c["pages"])
    pkv.attn_decode_step_noalloc(*args)  # warm-up: scratch lookup, code object load
    before = free_bytes()
    for _ in range(5):
        pkv.attn_decode_step_noalloc(*args)
    after = free_bytes()
    assert after == before, f"free device memory changed by {before - after} bytes"
