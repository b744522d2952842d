"""pkv_attn_prefill_split: prompt attention with each query tile's keys split
over several workgroups when the prompt's tiles leave CUs idle, then a merge
launch. Against the oracle within the attention tolerance (|got - want| <=
2e-3 + 1e-2 |want|); rows outside the prompts stay untouched; a grid that
covers the CUs (no split) gives pkv_attn_prefill's bytes.

parts() states the kernel's rule (the prompt's R query tiles x Hkv = w
workgroups split into max(2, CUs / w) ranges when w < CUs) so that each case
says which regime it covers."""
import numpy as np
import pytest
import torch

import oracle
import pkv
from _util import BS, close
from test_gpu_prefill import i16, i32, prefill_case

pytestmark = pytest.mark.gpu
SCALE = 1.0 / 16.0


def parts(c, G):
    """Key ranges per query tile the split kernel takes for case c."""
    bq = 32 if G >= 6 else 256 // G
    n = np.diff(c["cu"])
    R = int(sum((k + bq - 1) // bq for k in n if k > 1))
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    w = R * c["Hkv"]
    return 1 if w >= cus else max(2, cus // w)


def run_split(c, dev, workspace=True, init=0x3333):
    T, Hq, Hkv = c["T"], c["Hq"], c["Hkv"]
    out = torch.from_numpy(np.full((T, Hq, 256), init, np.uint16).view(np.int16)).to(dev)
    nbytes = pkv.attn_prefill_workspace(T, Hq, Hkv, c["seqs"])
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev) if workspace else None
    pkv.attn_prefill(i16(c["q"], dev), i16(c["kc"], dev), i16(c["vc"], dev), i16(c["qkv"], dev), c["qstride"], Hq,
                     Hkv, i32(c["pos"], dev), i32(c["cu"], dev), c["seqs"], i32(c["bt"], dev), c["max_blocks"], BS,
                     out, SCALE, None, 1, T, c["pages"], workspace=ws)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16), nbytes


def want_of(c, init=0x3333):
    return oracle.attn_prefill(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], c["Hq"], c["Hkv"], c["pos"], c["cu"],
                               c["seqs"], c["bt"], c["max_blocks"], BS, SCALE,
                               out=np.full((c["T"], c["Hq"], 256), init, np.uint16))


@pytest.mark.parametrize("G", [1, 2, 4, 6, 8])
@pytest.mark.parametrize("ctxs,chunks,seed", [
    ([3000], [20], 3),              # one short tile: up to 64 ranges of >= 4 key tiles
    ([2000], [300], 0),             # one chunk after a long context: 8 ranges per tile
    ([0], [700], 1),                # one prompt, causal tiles of every length
    ([100, 3000, 0], [70, 130, 33], 2),  # three chunks, ranges ending mid-tile
])
def test_split_prefill_matches_oracle(dev, G, ctxs, chunks, seed):
    print(f"case prefill split G={G} ctx={ctxs} chunk={chunks}", flush=True)
    c = prefill_case(ctxs, chunks, 4, 200 + seed, decode_rows=1, G=G)
    assert parts(c, G) > 1, "these shapes must split"
    got, _ = run_split(c, dev)
    assert (got[0] == 0x3333).all()  # the decode row is left to decode attention
    ok, err = close(got, want_of(c))
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("G", [2, 4, 8])
def test_split_prefill_beside_decode_rows(dev, G):
    """A chunk beside 60 one-token decode rows: the host's tile bound (60
    sequences) covers the CUs, the prompt's tiles do not, so the kernel
    splits; the decode rows are left to decode attention."""
    print(f"case prefill split beside decode rows G={G}", flush=True)
    c = prefill_case([2500], [200], 4, 280 + G, decode_rows=60, G=G)
    assert parts(c, G) > 1
    got, _ = run_split(c, dev)
    assert (got[:60] == 0x3333).all()
    ok, err = close(got, want_of(c))
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("G", [1, 4, 6])
def test_split_prefill_two_rounds_match_prefill(dev, G):
    """A 2,560-token prompt after 500 keys: R x Hkv between CUs / 2 and CUs
    at G = 4 (two ranges per tile, two rounds of workgroups). Against
    pkv_attn_prefill (itself pinned to the oracle) over the whole output,
    within the attention tolerance."""
    print(f"case prefill split two rounds G={G}", flush=True)
    c = prefill_case([500], [2560], 4, 290 + G, G=G)
    got, _ = run_split(c, dev)
    plain, _ = run_split(c, dev, workspace=False)
    ok, err = close(got, plain)
    assert ok, f"max |diff| {err}"


@pytest.mark.parametrize("split", [False, True])
def test_prefill_many_sequences_match_oracle(dev, split):
    """40 one-token decode sequences, then 30 short prompts (2-5 rows, so
    one tile each) at sequence indices 40-69: the kernels find their tiles
    64 sequences a round, and these tiles sit on both sides of the round
    boundary; through pkv_attn_prefill and pkv_attn_prefill_split."""
    print(f"case prefill many sequences split={split}", flush=True)
    ctxs = [50 + 37 * i for i in range(30)]
    chunks = [2 + i % 4 for i in range(30)]
    c = prefill_case(ctxs, chunks, 4, 300 + split, decode_rows=40, G=4)
    got, _ = run_split(c, dev, workspace=split)
    assert (got[:40] == 0x3333).all()
    ok, err = close(got, want_of(c))
    assert ok, f"max |diff| {err}"


def test_split_prefill_skips_spec_sequences(dev):
    """A verifying sequence (outs >= 0) is left to decode attention, as in
    pkv_attn_prefill (qwen35.cu:94-100)."""
    print("case prefill split spec rows", flush=True)
    c = prefill_case([500, 40], [90, 4], 4, 230, G=4)
    T, Hq = c["T"], c["Hq"]
    out = torch.from_numpy(np.full((T, Hq, 256), 0x3333, np.uint16).view(np.int16)).to(dev)
    ws = torch.empty(pkv.attn_prefill_workspace(T, Hq, 4, c["seqs"]), dtype=torch.uint8, device=dev)
    outs = np.full(2 * 4, -1, np.int32)  # [seqs][spec]: sequence 1 verifies drafts
    outs[4] = 0
    pkv.attn_prefill(i16(c["q"], dev), i16(c["kc"], dev), i16(c["vc"], dev), i16(c["qkv"], dev), c["qstride"], Hq, 4,
                     i32(c["pos"], dev), i32(c["cu"], dev), c["seqs"], i32(c["bt"], dev), c["max_blocks"], BS, out,
                     SCALE, i32(outs, dev), 4, T, c["pages"], workspace=ws)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    assert (got[90:] == 0x3333).all()
    want = oracle.attn_prefill(c["q"], c["kc"], c["vc"], c["qkv"], c["qstride"], Hq, 4, c["pos"], c["cu"],
                               c["seqs"], c["bt"], c["max_blocks"], BS, SCALE, outs=outs, spec=4,
                               out=np.full((T, Hq, 256), 0x3333, np.uint16))
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"


def test_split_prefill_rejects_a_short_workspace(dev):
    print("case prefill split short workspace", flush=True)
    c = prefill_case([2000], [300], 4, 240, G=4)
    T, Hq = c["T"], c["Hq"]
    need = pkv.attn_prefill_workspace(T, Hq, 4, c["seqs"])
    ws = torch.empty(need - 256, dtype=torch.uint8, device=dev)
    out = torch.zeros(T, Hq, 256, dtype=torch.int16, device=dev)
    with pytest.raises(pkv.PkvError) as e:
        pkv.attn_prefill(i16(c["q"], dev), i16(c["kc"], dev), i16(c["vc"], dev), i16(c["qkv"], dev), c["qstride"],
                         Hq, 4, i32(c["pos"], dev), i32(c["cu"], dev), c["seqs"], i32(c["bt"], dev), c["max_blocks"],
                         BS, out, SCALE, None, 1, T, c["pages"], workspace=ws)
    assert e.value.status == pkv.ERR_INVALID


def test_split_prefill_without_a_split_is_prefill(dev):
    """A prompt whose tiles cover the CUs is not split and gives the bytes of
    pkv_attn_prefill."""
    print("case prefill split none", flush=True)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    n = (cus // 4 + 8) * 64  # query tiles x 4 kv heads >= CUs
    c = prefill_case([0], [n], 4, 250, G=4)
    assert parts(c, 4) == 1
    got, _ = run_split(c, dev)
    plain, _ = run_split(c, dev, workspace=False)
    assert np.array_equal(got, plain)


def test_split_prefill_graph_replay_matches_eager(dev):
    """The split kernel and its merge captured into a HIP graph and replayed
    3 times (eager launches and synchronizations between) give the eager
    bytes each time."""
    print("case prefill split graph replay", flush=True)
    c = prefill_case([1500], [200], 4, 260, G=4)
    T, Hq = c["T"], c["Hq"]
    args = [i16(c[k], dev) for k in ("q", "kc", "vc", "qkv")]
    pos, cu, bt = i32(c["pos"], dev), i32(c["cu"], dev), i32(c["bt"], dev)
    ws = torch.empty(pkv.attn_prefill_workspace(T, Hq, 4, c["seqs"]), dtype=torch.uint8, device=dev)
    out = torch.zeros(T, Hq, 256, dtype=torch.int16, device=dev)

    def launch():
        pkv.attn_prefill(*args, c["qstride"], Hq, 4, pos, cu, c["seqs"], bt, c["max_blocks"], BS, out, SCALE, None,
                         1, T, c["pages"], workspace=ws)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        launch()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out.cpu().numpy().copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch()
    for r in range(3):
        if r % 2:
            launch()
            torch.cuda.synchronize()
        out.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager), f"replay {r}"


@pytest.mark.parametrize("G", [4, 6])
def test_split_prefill_e4m3_matches_oracle(dev, G):
    """pkv_attn_prefill_e4m3_split: a chunk after a long context over an
    E4M3 cache against the oracle."""
    print(f"case prefill e4m3 split G={G}", flush=True)
    from test_gpu_e4m3 import e4m3_cache
    c = prefill_case([3000, 0], [150, 90], 4, 270 + G, decode_rows=1, G=G)
    T, Hq = c["T"], c["Hq"]
    rng = np.random.default_rng(271 + G)
    k8, v8 = e4m3_cache(c["kc"].shape, rng), e4m3_cache(c["vc"].shape, rng)
    ks = (rng.random(c["kc"].shape[:2]) * 0.004 + 0.001).astype(np.float32)
    vs = (rng.random(c["vc"].shape[:2]) * 0.004 + 0.001).astype(np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16) if a.dtype == np.uint16
                                   else np.ascontiguousarray(a)).to(dev)
    init = np.full((T, Hq, 256), 0x3333, np.uint16)
    out = t(init.copy())
    assert parts(c, G) > 1
    nbytes = pkv.attn_prefill_workspace(T, Hq, 4, c["seqs"])
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    pkv.attn_prefill_e4m3(t(c["q"]), t(k8), t(v8), t(ks), t(vs), t(c["qkv"]), c["qstride"], Hq, 4, t(c["pos"]),
                          t(c["cu"]), c["seqs"], t(c["bt"]), c["max_blocks"], BS, out, SCALE, None, 1, T, c["pages"],
                          workspace=ws)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    want = oracle.attn_prefill8(c["q"], k8, v8, ks, vs, c["qkv"], c["qstride"], Hq, 4, c["pos"], c["cu"], c["seqs"],
                                c["bt"], c["max_blocks"], BS, SCALE, out=init.copy())
    assert (got[0] == 0x3333).all()
    ok, err = close(got, want)
    assert ok, f"max |diff| {err}"
