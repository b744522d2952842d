"""Seeded random sweep over the attention entry points: each case draws an
entry point (decode, verify, their E4M3 forms, the fused step, prompts
through the library (also with split keys) and through the code object,
bf16 and E4M3), a query-
head group G in {1, 2, 4, 6, 8}, a kv-head count, ragged lengths and a key-
range size, and compares the GPU result with the oracle within the north
star's tolerance (|got - want| <= 2e-3 + 1e-2 |want|; appended cache rows
bit for bit). The hand-picked tests cover each path's edges; this covers the
combinations between them. Every case prints its parameters first, so a
failure names its seed."""
import numpy as np
import pytest

import oracle
import pkv
from _util import BS, close, decode_case
from test_gpu_decode import run_gpu, run_oracle
from test_gpu_e4m3 import e4m3_cache, run_decode8
from test_gpu_groups import _prefill
from test_gpu_prefill import prefill_case
from test_gpu_step import oracle_step, run as run_step, step_case
from test_gpu_verify import run_oracle as run_oracle_v, run_verify, verify_case

pytestmark = pytest.mark.gpu
SCALE = 1.0 / 16.0
KINDS = ["decode", "verify", "decode8", "verify8", "step", "prefill", "prefill8", "prefill_ref", "prefill8_ref",
         "prefill_split"]


@pytest.fixture(autouse=True)
def default_config():
    pkv.attn_decode_config(1, 32)
    yield
    pkv.attn_decode_config(1, 32)


def draw(seed):
    """The case of one seed: kind, G, Hkv, min_range and lengths."""
    rng = np.random.default_rng(1000 + seed)
    kind = KINDS[seed % len(KINDS)]
    G = 4 if kind == "step" else int(rng.choice([1, 2, 4, 6, 8]))
    Hkv = int(rng.choice([1, 2, 4, 8] if G <= 4 else [1, 2, 4]))
    min_range = int(rng.choice([16, 32, 128, 1 << 20]))
    B = int(rng.integers(1, 25))
    short = rng.random() < 0.3  # many short contexts (pieces cross ranges often)
    lens = [int(x) for x in (rng.integers(1, 40, B) if short else rng.integers(1, 3000, B))]
    return rng, kind, G, Hkv, min_range, lens


def e4m3_of(c, rng, amp):
    """E4M3 bytes and per-(slot, kv head) scales in [0.001, 0.001 + amp) (the
    E4M3 tests' ranges: 0.02 for decode rows, 0.004 for prompts)."""
    k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
    ks = (rng.random(c["kc"].shape[:2]) * amp + 0.001).astype(np.float32)
    vs = (rng.random(c["vc"].shape[:2]) * amp + 0.001).astype(np.float32)
    return k8, v8, ks, vs


@pytest.mark.parametrize("seed", range(50))
def test_random_case_matches_oracle(dev, seed):
    rng, kind, G, Hkv, min_range, lens = draw(seed)
    print(f"case sweep seed={seed} kind={kind} G={G} Hkv={Hkv} min_range={min_range} lens={lens[:8]}"
          f"{'..' if len(lens) > 8 else ''} ({len(lens)} seqs)", flush=True)
    pkv.attn_decode_config(1, min_range)
    if kind in ("decode", "decode8"):
        c = decode_case(lens, G * Hkv, Hkv, seed)
        if kind == "decode":
            got, want = run_gpu(c, dev), run_oracle(c, cu=c["cu"])
        else:
            k8, v8, ks, vs = e4m3_of(c, rng, 0.02)
            got = run_decode8(c, k8, v8, ks, vs, dev)
            want = oracle.attn_decode8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], c["Hq"], Hkv, c["pos"],
                                       c["tok_seq"], c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"])
    elif kind in ("verify", "verify8"):
        groups = [(max(0, L - 8), int(rng.integers(1, 8))) for L in lens]
        c = verify_case(groups, Hkv, seed, G=G)
        if kind == "verify":
            got, want = run_verify(c, dev), run_oracle_v(c)
        else:
            k8, v8, ks, vs = e4m3_of(c, rng, 0.02)
            got = run_decode8(c, k8, v8, ks, vs, dev, entry="verify")
            want = oracle.attn_decode8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], c["Hq"], Hkv, c["pos"],
                                       c["tok_seq"], c["bt"], c["max_blocks"], BS, SCALE, cu=c["cu"])
    elif kind == "step":
        per_seq = int(rng.choice([1, 1, 2, 4]))
        c = step_case([max(L, per_seq) for L in lens], Hkv, seed, per_seq)
        got, kc, vc = run_step(c, dev, fused=True)
        want, wkc, wvc = oracle_step(c)
        assert np.array_equal(kc, wkc) and np.array_equal(vc, wvc), "appended rows differ"
    else:
        n = min(len(lens), 6)
        ctxs = [int(x) for x in rng.integers(0, 800, n)]
        chunks = [int(x) for x in rng.integers(1, 160, n)]
        c = prefill_case(ctxs, chunks, Hkv, seed, decode_rows=1, G=G)
        entry = "ref" if kind.endswith("_ref") else "lib"
        if kind == "prefill_split":
            from test_gpu_prefill_split import run_split, want_of
            got, _ = run_split(c, dev)
            want = want_of(c)
        elif kind.startswith("prefill8"):
            f8 = e4m3_of(c, rng, 0.004)
            got, init = _prefill(c, dev, entry, f8=f8)
            want = oracle.attn_prefill8(c["q"], f8[0], f8[1], f8[2], f8[3], c["qkv"], c["qstride"], c["Hq"], Hkv,
                                        c["pos"], c["cu"], c["seqs"], c["bt"], c["max_blocks"], BS, SCALE,
                                        out=init.copy())
        else:
            got, init = _prefill(c, dev, entry)
            want = oracle.attn_prefill(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], Hkv, c["pos"],
                                       c["cu"], c["seqs"], c["bt"], c["max_blocks"], BS, SCALE, out=init.copy())
        assert (got[0] == 0x3333).all(), "the decode row was written by prompt attention"
    ok, err = close(got, want)
    assert ok, f"seed {seed} ({kind}): max |diff| {err}"
