"""GPU parity: the fused decode step (the key-range kernel appends the step's
rows itself, then the merge: pkv_attn_decode_step) against the unfused
launches and the oracle, eager and replayed from a HIP graph.

The fused kernel computes the same partials in the same order as
pkv_append + pkv_attn_decode, so its outputs must be bit-identical to theirs;
the caches it writes must equal the oracle's append bit for bit; outputs are
within the north-star tolerance of the oracle (max-abs 2e-3, rel 1e-2)."""
import numpy as np
import pytest
import torch

import oracle
import pkv
from _util import BS, D, bf16_bits, close, decode_case

pytestmark = pytest.mark.gpu
SCALE = 1.0 / 16.0


def i16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


def i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)


@pytest.fixture(autouse=True)
def default_config():
    pkv.attn_decode_config(1, 32)
    yield
    pkv.attn_decode_config(1, 32)


def step_case(lens, Hkv, seed, per_seq=1, G=4):
    """A step in which every sequence feeds `per_seq` new tokens (decode,
    or verification of per_seq - 1 drafts) at consecutive positions ending at
    len - 1; their K/V rows come from qkv rows like the reference's layout.
    G query heads per kv head."""
    Hq = G * Hkv
    c = decode_case(lens, Hq, Hkv, seed)
    rng = np.random.default_rng(seed + 100)
    B = len(lens)
    pos = np.concatenate([np.arange(L - per_seq, L) for L in lens]).astype(np.int32)
    tok_seq = np.repeat(np.arange(B), per_seq).astype(np.int32)
    T = len(pos)
    slot = (c["bt"][tok_seq, pos // BS] * BS + pos % BS).astype(np.int32)
    qkv = bf16_bits(rng.standard_normal((T, c["qstride"])) * 0.5)
    q = bf16_bits(rng.standard_normal((T, Hq, D)) * 0.5)
    cu = (np.arange(B + 1) * per_seq).astype(np.int32)
    outs = np.full(B, 0 if per_seq > 1 else -1, np.int32)
    return dict(c, q=q, qkv=qkv, pos=pos, tok_seq=tok_seq, cu=cu, slot=slot, T=T, outs=outs, Hq=Hq, Hkv=Hkv)


def run(c, dev, fused, repeat=1):
    Hq, Hkv, T = c["Hq"], c["Hkv"], c["T"]
    kc, vc = i16(c["kc"], dev), i16(c["vc"], dev)
    q, qkv = i16(c["q"], dev), i16(c["qkv"], dev)
    pos, ts, bt, cu, slot = (i32(c[k], dev) for k in ("pos", "tok_seq", "bt", "cu", "slot"))
    outs = i32(c["outs"], dev)
    out = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev)
    ws = torch.empty(pkv.attn_decode_workspace(T, Hq), dtype=torch.uint8, device=dev)
    k_rows = qkv.data_ptr() + 2 * (2 * Hq * D)
    v_rows = k_rows + 2 * Hkv * D
    stride = c["qstride"] * 2
    for _ in range(repeat):
        if fused:
            pkv.attn_decode_step(k_rows, v_rows, stride, slot, q, kc, vc, qkv, c["qstride"], Hq, Hkv, pos, ts, bt,
                                 c["max_blocks"], BS, out, SCALE, cu, 0, outs, 1, T, c["pages"], ws)
        else:
            pkv.append(k_rows, v_rows, stride, slot, T, Hkv, D * 2, kc, vc, c["pages"] * BS)
            pkv.attn_decode(q, kc, vc, qkv, c["qstride"], Hq, Hkv, pos, ts, bt, c["max_blocks"], BS, out, SCALE, cu,
                            0, outs, 1, T, c["pages"], ws)
    torch.cuda.synchronize()
    return (out.cpu().numpy().view(np.uint16), kc.cpu().numpy().view(np.uint16), vc.cpu().numpy().view(np.uint16))


def oracle_step(c):
    kc, vc = c["kc"].copy(), c["vc"].copy()
    Hq, Hkv = c["Hq"], c["Hkv"]
    k_rows = np.ascontiguousarray(c["qkv"][:, 2 * Hq * D:2 * Hq * D + Hkv * D])
    v_rows = np.ascontiguousarray(c["qkv"][:, 2 * Hq * D + Hkv * D:2 * Hq * D + 2 * Hkv * D])
    oracle.append(k_rows, v_rows, c["slot"], kc, vc)
    out, _ = oracle.attn_decode(c["q"], kc, vc, c["qkv"], c["qstride"], Hq, Hkv, c["pos"], c["tok_seq"], c["bt"],
                                c["max_blocks"], BS, SCALE, cu=c["cu"], skip_prompts=0, outs=c["outs"], spec=1)
    return out, kc, vc


@pytest.mark.parametrize("lens,Hkv,per_seq,seed", [
    ([1, 2, 17, 33, 700, 4097], 4, 1, 0),      # decode rows, first key fresh for len 1
    ([3000, 5000, 100, 8193], 4, 1, 1),
    ([900, 1200, 64], 4, 4, 2),                # verify rows: 4 fresh tokens per sequence
    ([50] * 30, 4, 2, 3),                      # many short sequences, 2 fresh each
    ([2000, 3000], 8, 1, 4),                   # two kv-head groups
])
def test_fused_step_matches_unfused_and_oracle(dev, lens, Hkv, per_seq, seed):
    print(f"case step lens={lens[:6]} Hkv={Hkv} per_seq={per_seq}", flush=True)
    c = step_case(lens, Hkv, seed, per_seq)
    f_out, f_kc, f_vc = run(c, dev, fused=True)
    u_out, u_kc, u_vc = run(c, dev, fused=False)
    o_out, o_kc, o_vc = oracle_step(c)
    assert np.array_equal(f_kc, o_kc) and np.array_equal(f_vc, o_vc), "fused append differs from the oracle"
    assert np.array_equal(u_kc, o_kc) and np.array_equal(u_vc, o_vc)
    assert np.array_equal(f_out, u_out), "fused and unfused outputs differ"
    ok, err = close(f_out, o_out)
    assert ok, err


@pytest.mark.parametrize("lens,Hkv,per_seq,G,seed", [
    ([1, 2, 17, 33, 700, 4097], 4, 1, 6, 20),  # the reference's 27B shape (24 q / 4 kv heads)
    ([900, 1200, 64, 3], 4, 2, 6, 21),         # 2 fresh tokens per sequence: a whole 2-row segment
    ([3000, 77, 8193], 4, 3, 6, 22),           # 3 fresh: a 2-row segment and a 1-row one
    ([2000, 3000, 15], 8, 1, 6, 23),           # two kv-head groups
    ([500, 16, 4100], 4, 2, 8, 24),
    ([500, 16, 4100], 4, 4, 2, 25),
    ([500, 16, 4100], 4, 1, 1, 26),
])
def test_fused_step_other_groups(dev, lens, Hkv, per_seq, G, seed):
    """The fused step for G != 4 (the verify kernel with the append fused in,
    then the verify merge): caches bit-exact against the oracle's append,
    outputs bit-identical to pkv_append + pkv_attn_decode (the same kernel
    body reading the cache), within tolerance of the oracle."""
    print(f"case step G={G} lens={lens} Hkv={Hkv} per_seq={per_seq}", flush=True)
    c = step_case(lens, Hkv, seed, per_seq, G=G)
    f_out, f_kc, f_vc = run(c, dev, fused=True)
    u_out, u_kc, u_vc = run(c, dev, fused=False)
    o_out, o_kc, o_vc = oracle_step(c)
    assert np.array_equal(f_kc, o_kc) and np.array_equal(f_vc, o_vc), "fused append differs from the oracle"
    assert np.array_equal(u_kc, o_kc) and np.array_equal(u_vc, o_vc)
    assert np.array_equal(f_out, u_out), "fused and unfused outputs differ"
    ok, err = close(f_out, o_out, what=f"fused step G={G}")
    assert ok, err


def test_fused_step_g6_c3_full_size(dev):
    """C3 at the 27B shape (batch 64, contexts U[512, 8192], 24 q / 4 kv
    heads, a 65,536-page pool): the fused step equals append + decode bit for
    bit on every row and writes the same caches; 8 sequences against the
    oracle."""
    from pkv import synth
    from _util import bits, host_pages, oracle_decode_rows
    print("case step G=6 c3 full", flush=True)
    Hq, Hkv, pages = 24, 4, 65536
    lens = synth.c3_lengths(seed=31)
    meta = synth.decode_meta(lens, pages, steps=1, seed=31)
    st = meta.step(0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(31)
    kc = (torch.randn(pages * BS, Hkv, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    vc = (torch.randn(pages * BS, Hkv, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    B = meta.B
    q = (torch.randn(B, Hq, D, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    qstride = synth.qkv_stride(Hq, Hkv)
    qkv = (torch.randn(B, qstride, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
    pos, ts, cu = i32(st["pos"], dev), i32(st["tok_seq"], dev), i32(st["cu"], dev)
    slot, bt = i32(st["slot_map"], dev), i32(meta.block_table, dev)
    ws = torch.empty(pkv.attn_decode_workspace(B, Hq), dtype=torch.uint8, device=dev)
    k_rows = qkv.data_ptr() + 2 * (2 * Hq * D)
    v_rows = k_rows + 2 * Hkv * D
    kc0, vc0 = kc.clone(), vc.clone()
    out_f = torch.zeros(B, Hq, D, dtype=torch.bfloat16, device=dev)
    pkv.attn_decode_step(k_rows, v_rows, qstride * 2, slot, q, kc, vc, qkv, qstride, Hq, Hkv, pos, ts, bt,
                         meta.max_blocks, BS, out_f, SCALE, cu, 0, None, 1, B, pages, ws)
    out_u = torch.zeros_like(out_f)
    pkv.append(k_rows, v_rows, qstride * 2, slot, B, Hkv, D * 2, kc0, vc0, pages * BS)
    pkv.attn_decode(q, kc0, vc0, qkv, qstride, Hq, Hkv, pos, ts, bt, meta.max_blocks, BS, out_u, SCALE, cu, 0, None,
                    1, B, pages, ws)
    torch.cuda.synchronize()
    assert torch.equal(kc.view(torch.int16), kc0.view(torch.int16)) and torch.equal(vc.view(torch.int16),
                                                                                  vc0.view(torch.int16))
    assert torch.equal(out_f.view(torch.int16), out_u.view(torch.int16)), "fused and unfused outputs differ"
    del kc0, vc0
    sel = np.arange(0, B, 8)
    need = (st["pos"][sel] + BS) // BS
    kc_h, vc_h, bt_h, _ = host_pages(kc, vc, meta.block_table[sel], need)
    want = oracle_decode_rows(bits(q)[sel], kc_h, vc_h, bits(qkv)[sel], qstride, Hq, Hkv, st["pos"][sel],
                              np.arange(len(sel), dtype=np.int32), bt_h, meta.max_blocks, SCALE)
    ok, err = close(bits(out_f)[sel], want, what="c3 G=6 fused step, 8 of 64 sequences")
    assert ok, err


def test_fused_step_repeated_calls_are_idempotent(dev):
    """Ten calls in a row on the same workspace (re-appending the same rows)
    give identical outputs; a finer range split stays within tolerance."""
    print("case step repeat", flush=True)
    c = step_case([5000, 3000, 1000, 40], 4, 5)
    once, _, _ = run(c, dev, fused=True, repeat=1)
    many, _, _ = run(c, dev, fused=True, repeat=10)
    assert np.array_equal(once, many)
    pkv.attn_decode_config(1, 16)  # more ranges per token
    finer, _, _ = run(c, dev, fused=True, repeat=3)
    ok, err = close(finer, once)
    assert ok, err


def test_fused_step_many_one_key_sequences(dev):
    """16,400 one-key sequences (every key is the step's own): fused equals
    unfused, and the output is the closed form of a single key."""
    print("case step many tokens", flush=True)
    B = 16400
    c = step_case([1] * B, 1, 6)
    f_out, f_kc, _ = run(c, dev, fused=True)
    u_out, u_kc, _ = run(c, dev, fused=False)
    assert np.array_equal(f_out, u_out) and np.array_equal(f_kc, u_kc)
    # one key: the output is bf16(rbf(v) * sigmoid(gate))
    v = oracle.b2f(c["qkv"][:, 2 * 4 * D + D:2 * 4 * D + 2 * D])  # V rows, Hkv = 1
    gate = oracle.b2f(c["qkv"][:, :4 * 2 * D].reshape(B, 4, 2, D)[:, :, 1, :])
    want = bf16_bits(v[:, None, :] / (np.float32(1) + np.exp(-gate, dtype=np.float32)))
    ok, err = close(f_out, want)
    assert ok, err


@pytest.mark.parametrize("G", [4, 6])
def test_step_graph_replay_matches_eager(dev, G):
    """The step captured into a HIP graph (torch.cuda.CUDAGraph) and replayed
    5 times, with eager launches and synchronizations in between, reproduces
    the eager outputs and caches bit for bit each time (G = 6: the verify
    kernel's fused step)."""
    print(f"case step graph replay G={G}", flush=True)
    c = step_case([4000, 900, 6000, 33], 4, 7, G=G)
    Hq, Hkv, T = c["Hq"], c["Hkv"], c["T"]
    eager_out, eager_kc, _ = run(c, dev, fused=True)
    kc, vc = i16(c["kc"], dev), i16(c["vc"], dev)
    q, qkv = i16(c["q"], dev), i16(c["qkv"], dev)
    pos, ts, bt, cu, slot = (i32(c[k], dev) for k in ("pos", "tok_seq", "bt", "cu", "slot"))
    out = torch.zeros(T, Hq, D, dtype=torch.int16, device=dev)
    ws = torch.empty(pkv.attn_decode_workspace(T, Hq), dtype=torch.uint8, device=dev)
    k_rows = qkv.data_ptr() + 2 * (2 * Hq * D)
    v_rows = k_rows + 2 * Hkv * D

    def launch():
        pkv.attn_decode_step(k_rows, v_rows, c["qstride"] * 2, slot, q, kc, vc, qkv, c["qstride"], Hq, Hkv, pos, ts,
                             bt, c["max_blocks"], BS, out, SCALE, cu, 0, None, 1, T, c["pages"], ws)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        launch()  # warm up outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch()
    for r in range(5):
        out.fill_(0)
        launch() if r % 2 else None  # eager work between replays
        torch.cuda.synchronize()
        out.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint16), eager_out), f"replay {r}"
        assert np.array_equal(kc.cpu().numpy().view(np.uint16), eager_kc)


def test_padded_bucket_graph_replay_through_meta_buffer(dev):
    """Graph-bucket integration (engine.rs:704-720): the step's arrays live in
    one int32 buffer at the reference's Meta offsets (pkv_meta_layout,
    model.rs:1245-1354); a step of 5 sequences is padded to the bucket of 8
    with Scheduler::pad's rows (pkv_kv_pad: slot -1, position 0, block table
    row 0), captured once into a HIP graph and replayed for two different
    steps with the buffer's contents rewritten. Real rows match the oracle;
    padding rows write no KV (caches equal the oracle's append bit for bit)."""
    print("case padded bucket graph replay", flush=True)
    Hkv, Hq, bucket, maxb = 4, 16, 8, 600
    lay = pkv.meta_layout(bucket, bucket, maxb, 1)
    meta_d = torch.zeros(lay["words"], dtype=torch.int32, device=dev)
    ptr = lambda name: meta_d.data_ptr() + 4 * lay[name]
    lens0 = [4000, 900, 6000, 33, 1500]
    base = decode_case([L + 1 for L in lens0], Hq, Hkv, 21, pages=2400)
    kc, vc = i16(base["kc"], dev), i16(base["vc"], dev)
    kc_ref, vc_ref = base["kc"].copy(), base["vc"].copy()
    qstride = base["qstride"]
    q_d = torch.zeros(bucket, Hq, D, dtype=torch.int16, device=dev)
    qkv_d = torch.zeros(bucket, qstride, dtype=torch.int16, device=dev)
    out = torch.zeros(bucket, Hq, D, dtype=torch.int16, device=dev)
    ws = torch.empty(pkv.attn_decode_workspace(bucket, Hq), dtype=torch.uint8, device=dev)
    k_rows = qkv_d.data_ptr() + 2 * (2 * Hq * D)
    v_rows = k_rows + 2 * Hkv * D

    def host_step(k):
        """Step k: every sequence feeds token lens0 + k; arrays padded to the bucket."""
        lens = [L + k + 1 for L in lens0]
        m = {n: np.zeros(sz, np.int32) for n, sz in (("pos", bucket), ("slot_map", bucket), ("tok_seq", bucket),
                                                     ("cu", bucket + 1), ("limits", bucket))}
        m["block_table"] = np.zeros((bucket, maxb), np.int32)
        for s, L in enumerate(lens):
            p = L - 1
            m["pos"][s] = p
            m["tok_seq"][s] = s
            m["cu"][s + 1] = s + 1
            m["block_table"][s, :base["max_blocks"]] = base["bt"][s]
            m["slot_map"][s] = base["bt"][s][p // BS] * BS + p % BS
            m["limits"][s] = ((L + BS - 1) // BS) * BS - 1
        pkv.pad_rows(m, len(lens), bucket, 1)
        rng = np.random.default_rng(100 + k)
        q = bf16_bits(rng.standard_normal((bucket, Hq, D)) * 0.5)
        qkv = bf16_bits(rng.standard_normal((bucket, qstride)) * 0.5)
        return lens, m, q, qkv

    def upload(m, q, qkv):
        staging = np.zeros(lay["words"], np.int32)
        for n in ("pos", "slot_map", "tok_seq", "cu", "limits"):
            staging[lay[n]:lay[n] + len(m[n])] = m[n]
        staging[lay["block_table"]:lay["block_table"] + m["block_table"].size] = m["block_table"].ravel()
        meta_d.copy_(torch.from_numpy(staging))
        q_d.copy_(i16(q, dev))
        qkv_d.copy_(i16(qkv, dev))

    def launch():
        pkv.attn_decode_step(k_rows, v_rows, qstride * 2, ptr("slot_map"), q_d, kc, vc, qkv_d, qstride, Hq, Hkv,
                             ptr("pos"), ptr("tok_seq"), ptr("block_table"), maxb, BS, out, SCALE, ptr("cu"), 0, None,
                             1, bucket, base["pages"], ws)

    def check(k):
        lens, m, q, qkv = host_step(k)
        S = len(lens)
        # the oracle's append of the real rows, then attention over the updated cache
        for s in range(S):
            slot = m["slot_map"][s]
            kc_ref[slot] = qkv[s, 2 * Hq * D:2 * Hq * D + Hkv * D].reshape(Hkv, D)
            vc_ref[slot] = qkv[s, 2 * Hq * D + Hkv * D:2 * Hq * D + 2 * Hkv * D].reshape(Hkv, D)
        want, _ = oracle.attn_decode(q[:S], kc_ref, vc_ref, qkv[:S], qstride, Hq, Hkv, m["pos"][:S],
                                     m["tok_seq"][:S], m["block_table"][:S], maxb, BS, SCALE)
        got = out.cpu().numpy().view(np.uint16)[:S]
        ok, err = close(got, want)
        assert ok, f"step {k}: max |diff| {err}"
        assert np.array_equal(kc.cpu().numpy().view(np.uint16), kc_ref), f"step {k}: K cache"
        assert np.array_equal(vc.cpu().numpy().view(np.uint16), vc_ref), f"step {k}: V cache"

    upload(*host_step(0)[1:])
    s_ = torch.cuda.Stream()
    s_.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s_):
        launch()  # warm-up outside capture (step 0, eager)
    torch.cuda.current_stream().wait_stream(s_)
    torch.cuda.synchronize()
    check(0)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch()
    for k in (1, 2):
        upload(*host_step(k)[1:])
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        check(k)
