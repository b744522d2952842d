"""Block-table entries past a sequence's last page are never read. The
engine's tables (Meta block_table, src/model.rs:1245-1354) hold whatever an
earlier step left there beyond a sequence's ceil(len / 16) pages (padding rows
get 0, sched.rs:1219-1261, but a shrinking sequence keeps stale ids), so
every entry point must give the same bytes when those entries hold garbage:
ids past the pool, negative ids, the largest int32."""
import numpy as np
import pytest

import pkv
from _util import BS, decode_case
from test_gpu_decode import run_gpu
from test_gpu_e4m3 import e4m3_cache, run_decode8
from test_gpu_groups import _prefill
from test_gpu_prefill import prefill_case
from test_gpu_step import run as run_step, step_case
from test_gpu_verify import run_verify, verify_case

pytestmark = pytest.mark.gpu
GARBAGE = np.array([2**31 - 1, -5, 1 << 28, -(2**31), 70000], np.int64)


def with_garbage(c, used):
    """c with every block-table entry past used[s] pages of row s replaced by
    garbage ids."""
    bt = c["bt"].copy()
    for s in range(bt.shape[0]):
        n = bt.shape[1] - used[s]
        bt[s, used[s]:] = np.resize(GARBAGE, n).astype(np.int32)
    return dict(c, bt=bt)


def pages_of(lens):
    return [(L + BS - 1) // BS for L in lens]


@pytest.fixture(autouse=True)
def default_config():
    pkv.attn_decode_config(1, 32)
    yield
    pkv.attn_decode_config(1, 32)


@pytest.mark.parametrize("G", [4, 6])
def test_decode_ignores_entries_past_the_last_page(dev, G):
    print(f"case tables decode G={G}", flush=True)
    lens = [17, 4000, 1, 700, 64, 2049]
    c = decode_case(lens, G * 4, 4, 110 + G)
    assert c["bt"].shape[1] > min(pages_of(lens))
    want = run_gpu(c, dev)
    assert np.array_equal(run_gpu(with_garbage(c, pages_of(lens)), dev), want)


def test_verify_ignores_entries_past_the_last_page(dev):
    print("case tables verify", flush=True)
    groups = [(300, 4), (0, 3), (2000, 5), (40, 2)]
    c = verify_case(groups, 4, 120)
    want = run_verify(c, dev)
    got = run_verify(with_garbage(c, pages_of([L0 + n for L0, n in groups])), dev)
    assert np.array_equal(got, want)


def test_step_ignores_entries_past_the_last_page(dev):
    print("case tables fused step", flush=True)
    lens = [33, 5000, 2, 900]
    c = step_case(lens, 4, 130)
    want, wkc, _ = run_step(c, dev, fused=True)
    got, gkc, _ = run_step(with_garbage(c, pages_of(lens)), dev, fused=True)
    assert np.array_equal(got, want) and np.array_equal(gkc, wkc)


def test_e4m3_decode_ignores_entries_past_the_last_page(dev):
    print("case tables decode e4m3", flush=True)
    lens = [17, 3000, 1, 500]
    c = decode_case(lens, 16, 4, 140)
    rng = np.random.default_rng(141)
    k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
    ks = (rng.random(c["kc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    vs = (rng.random(c["vc"].shape[:2]) * 0.02 + 0.001).astype(np.float32)
    want = run_decode8(c, k8, v8, ks, vs, dev)
    assert np.array_equal(run_decode8(with_garbage(c, pages_of(lens)), k8, v8, ks, vs, dev), want)


@pytest.mark.parametrize("entry", ["lib", "ref"])
def test_prefill_ignores_entries_past_the_last_page(dev, entry):
    """Prompt attention (the library's kernel, and the code object's, which
    does not clamp ids: the reference ABI passes no pool size)."""
    print(f"case tables prefill {entry}", flush=True)
    ctxs, chunks = [100, 0, 700], [70, 33, 130]
    c = prefill_case(ctxs, chunks, 4, 150, decode_rows=1)
    lens = [40] + [x + n for x, n in zip(ctxs, chunks)]  # the decode row's sequence first (40 keys)
    want, _ = _prefill(c, dev, entry)
    got, _ = _prefill(with_garbage(c, pages_of(lens)), dev, entry)
    assert np.array_equal(got, want)
