"""Host KV manager (libpkv pkv_kv_*) against the reference scheduler's own
tests restated at the KV level (src/sched.rs:1473-1780) and against
invariants: reference counts equal the table and cache-entry occurrences,
free pages are exactly the unreferenced ones, copy-on-write never leaves a
page shared by a writer, truncation keeps what it keeps. CPU only."""
import numpy as np
import pytest

import pkv

BS = 16


def test_prefixes_are_kept_reused_and_evicted():
    """sched.rs:1563-1622 at the KV level: a 150-token prompt with 2 new
    tokens reserves 10 blocks; its 128-token entry keeps 8; after release
    64 - 8 are free; a 250-token prompt with the same start reuses 128 tokens
    and takes 8 more; its 192-token entry shares the first's 8 (64 - 12 free
    after release); a request needing every block evicts both entries."""
    kv = pkv.Kv(64, BS, max_entries=2)
    base = list(range(1, 151))
    a, cached = kv.admit(base, 2)
    assert cached == 0 and len(kv.blocks(a)) == 10
    kv.set_len(a, 150)
    kv.cache_add(a, base[:128])
    kv.release(a)
    assert kv.free_count() == 64 - 8
    longer = base + list(range(500, 600))
    assert kv.lookup(longer) == 128
    b, cached = kv.admit(longer, 1)
    assert cached == 128 and kv.len(b) == 128
    assert len(kv.blocks(b)) == 16  # ceil(251 / 16), the first 8 shared
    kv.set_len(b, 250)
    kv.cache_add(b, longer[:192])
    kv.release(b)
    assert kv.free_count() == 64 - 12
    c, cached = kv.admit(list(range(900, 1000)), 64 * 16 - 100)
    assert cached == 0 and kv.free_count() == 0 and kv.entries() == 0


def test_prompts_sharing_everything_before_the_last_message_reuse_it():
    """sched.rs:1524-1561: entries at 192 (the unit before the last
    message) and 256; a second prompt with the same first 200 tokens + turn
    token reuses 192 tokens."""
    kv = pkv.Kv(64, BS, max_entries=4)
    ask = lambda q: list(range(1, 201)) + [999] + list(range(q, q + 100))
    p1 = ask(1000)
    s1, _ = kv.admit(p1, 1)
    kv.set_len(s1, len(p1))
    for at in (192, 256):
        kv.cache_add(s1, p1[:at])
    kv.release(s1)
    p2 = ask(2000)
    s2, cached = kv.admit(p2, 1)
    assert cached == 192


def test_metadata_describes_paged_positions():
    """sched.rs:1641-1667: an 18-token prompt whose first step feeds 16
    tokens fills exactly the first block; the next chunk starts at bt[1]*16."""
    kv = pkv.Kv(64, BS)
    s, _ = kv.admit(list(range(1, 19)), 4)
    m = kv.fill([(s, 16)], max_tokens=16, max_blocks=8)
    assert list(m["pos"][:3]) == [0, 1, 2] and m["cu"][1] == 16
    first = m["block_table"][0, 0]
    assert m["slot_map"][15] == first * BS + 15
    kv.set_len(s, 16)
    m = kv.fill([(s, 2)], max_tokens=16, max_blocks=8)
    assert m["pos"][0] == 16 and m["slot_map"][0] == m["block_table"][0, 1] * BS
    assert m["limits"][0] == len(kv.blocks(s)) * BS - 1


def test_admission_reserves_the_whole_request():
    """sched.rs:1687-1697: 2 blocks hold one request of 20 + 12 tokens; the
    next must wait."""
    kv = pkv.Kv(2, BS)
    kv.admit(list(range(1, 21)), 12)
    with pytest.raises(pkv.PkvError) as e:
        kv.admit(list(range(1, 5)), 4)
    assert e.value.status == pkv.ERR_NO_BLOCKS


def test_release_frees_capacity():
    """sched.rs:1669-1685: a finished request's blocks return to the pool."""
    kv = pkv.Kv(64, BS)
    s, _ = kv.admit(list(range(1, 5)), 10)
    assert kv.free_count() == 63
    kv.release(s)
    assert kv.free_count() == 64


def test_padding_rows_point_nowhere():
    """sched.rs:1770-1779 / pad (:1219-1261): padding rows write no KV
    (slot -1), limits -1, block table rows 0, cu advancing by n."""
    kv = pkv.Kv(64, BS)
    m = kv.fill([], max_tokens=8, max_blocks=4, max_rows=4)
    pkv.pad_rows(m, 0, 3, 1)
    assert list(m["cu"][:4]) == [0, 1, 2, 3] and m["slot_map"][1] == -1
    assert (m["limits"][:3] == -1).all() and (m["block_table"][:3] == 0).all()
    with pytest.raises(pkv.PkvError):
        pkv.pad_rows(m, 0, 5, 1)  # more rows than the arrays hold


def test_copy_on_write_of_a_shared_partial_page():
    """A 40-token prefix (2 full pages + 8 slots of a third) shared by two
    sequences: the first write into the partial page copies it for the
    writer; the full pages stay shared; the reader keeps the original."""
    kv = pkv.Kv(16, BS)
    a = kv.new_seq()
    kv.reserve(a, 40)
    kv.set_len(a, 40)
    b = kv.new_seq()
    kv.share(b, a, 40)
    pa, pb = kv.blocks(a), kv.blocks(b)
    assert pa == pb and all(kv.refs(p) == 2 for p in pa)
    src, dst = kv.prepare_write(b, 40, 1)
    assert src == [pa[2]] and len(dst) == 1 and dst[0] not in pa
    assert kv.blocks(b) == pa[:2] + dst and kv.refs(pa[2]) == 1 and kv.refs(dst[0]) == 1
    # writing further into b's own page copies nothing; a's own write copies nothing either
    assert kv.prepare_write(b, 41, 5) == ([], [])
    assert kv.prepare_write(a, 40, 1) == ([], [])
    # writing past the table grows it
    assert kv.prepare_write(b, 48, 20) == ([], []) and len(kv.blocks(b)) == 5


def test_truncate_keeps_or_frees_pages():
    """Rollback of rejected drafts: reserve mode keeps pages (as the
    reference does); on-demand mode frees pages wholly past the new length."""
    kv = pkv.Kv(32, BS)
    s, _ = kv.admit(list(range(1, 100)), 60)  # 159 tokens -> 10 pages
    kv.set_len(s, 140)
    free0 = kv.free_count()
    kv.truncate(s, 137)
    assert kv.len(s) == 137 and kv.free_count() == free0 and len(kv.blocks(s)) == 10
    kv.truncate(s, 100, free_pages=True)
    assert len(kv.blocks(s)) == 7 and kv.free_count() == free0 + 3
    with pytest.raises(pkv.PkvError):
        kv.truncate(s, 101)  # cannot grow


def test_random_operations_keep_refcounts_consistent():
    rng = np.random.default_rng(0)
    kv = pkv.Kv(256, BS, max_entries=3)
    live = []
    for it in range(600):
        op = rng.integers(0, 6)
        try:
            if op == 0:
                prompt = list(rng.integers(1, 4, size=int(rng.integers(2, 300))))
                s, cached = kv.admit(prompt, int(rng.integers(0, 40)))
                kv.set_len(s, max(cached, len(prompt) - 1))
                live.append((s, prompt))
            elif op == 1 and live:
                s, prompt = live[int(rng.integers(0, len(live)))]
                u = (min(kv.len(s), len(prompt)) // 64) * 64
                if u >= 64:
                    kv.cache_add(s, prompt[:u])
            elif op == 2 and live:
                s, _ = live.pop(int(rng.integers(0, len(live))))
                kv.release(s)
            elif op == 3 and live:
                s, _ = live[int(rng.integers(0, len(live)))]
                n = kv.len(s)
                kv.prepare_write(s, n, int(rng.integers(1, 20)))
                kv.set_len(s, n + 1)
            elif op == 4 and live:
                s, _ = live[int(rng.integers(0, len(live)))]
                kv.truncate(s, int(rng.integers(0, kv.len(s) + 1)), bool(rng.integers(0, 2)))
            elif op == 5 and live:
                s, _ = live[int(rng.integers(0, len(live)))]
                d = kv.new_seq()
                kv.share(d, s, kv.len(s))
                live.append((d, []))
        except pkv.PkvError as e:
            assert e.status == pkv.ERR_NO_BLOCKS
        # invariant: table refs <= refcount, free pages have refcount 0
        counts = {}
        for s, _ in live:
            for b in kv.blocks(s):
                counts[b] = counts.get(b, 0) + 1
        for b, c in counts.items():
            assert kv.refs(b) >= c
        assert sum(1 for b in range(256) if kv.refs(b) == 0) == kv.free_count()
    for s, _ in live:
        kv.release(s)
    while kv.evict_one():
        pass
    assert kv.free_count() == 256


def test_meta_layout_regions_follow_the_reference_order():
    """pkv_meta_layout: the regions of Meta (model.rs:1245-1354) in order,
    each as long as the reference documents (per token: ids, pos, slot_map,
    tok_seq, emb_src, 3 rope rows, mtp_ids, mtp_src; cu and ocu: seqs + 1;
    per output row (seqs x spec): outs, last, temps, seeds, top_ks, top_ps,
    min_ps, masks, pen_cu + 1; snaps 4 per sequence; lora 1 + 3 per tile of
    16 tokens), laid end to end from 0 to words."""
    for T, S, B, spec in ((256, 64, 512, 1), (260, 32, 8192, 5), (4, 1, 1, 1)):
        lay = pkv.meta_layout(T, S, B, spec)
        O = S * spec
        tiles = T // 16 + S
        regions = [("ids", T), ("pos", T), ("slot_map", T), ("tok_seq", T), ("emb_src", T), ("rope", 3 * T),
                   ("mtp_ids", T), ("mtp_src", T), ("cu", S + 1), ("slots", S), ("fresh", S), ("outs", O),
                   ("ocu", S + 1), ("last", O), ("temps", O), ("seeds", O), ("top_ks", O), ("top_ps", O),
                   ("min_ps", O), ("pen_cu", O + 1), ("limits", S), ("snaps", 4 * S), ("block_table", S * B),
                   ("lora", 1 + 3 * tiles), ("masks", O)]
        at = 0
        for name, n in regions:
            assert lay[name] == at, (T, S, B, spec, name)
            at += n
        assert lay["words"] == at
    with pytest.raises(RuntimeError):
        pkv.meta_layout(0, 1, 1, 1)


@pytest.mark.parametrize("prefix", [16384, 16392])
def test_c4_plan_through_the_manager(prefix):
    """Config 4's tables as bench.py and the GPU test build them: a whole-unit
    prefix reaches the 8 sequences through the prefix cache (admission
    hits it), a prefix ending inside a page through sharing plus one
    copy-on-write per sequence; either way the prefix's whole pages end at
    refs 9 (entry + 8 sequences) once the seed is released."""
    from pkv import synth
    B, N = 8, 2048
    per_seq = (prefix + N + 15) // 16
    kv = pkv.Kv((prefix + 15) // 16 + B * (per_seq - prefix // 16) + 16, 16)
    plan = synth.c4_kv_plan(kv, prefix, N, B, seed=5)
    st, seed_blocks = plan["step"], plan["seed_blocks"]
    whole = seed_blocks[:prefix // 16]
    assert plan["via_cache"] == (prefix % 64 == 0)
    assert len(plan["cow"]) == (0 if prefix % 16 == 0 else B)
    assert all(kv.refs(b) == B + 1 for b in whole)
    assert list(st["cu"][:B + 1]) == [i * N for i in range(B + 1)]
    for s in range(B):
        assert (st["block_table"][s, :len(whole)] == whole).all()
        rows = slice(s * N, (s + 1) * N)
        assert (st["pos"][rows] == np.arange(prefix, prefix + N)).all()
        p = st["pos"][rows]
        assert (st["slot_map"][rows] == st["block_table"][s, p // 16] * 16 + p % 16).all()
    for src, dst in plan["cow"]:
        assert src == seed_blocks[-1] and kv.refs(dst) == 1
    if plan["cow"]:
        assert kv.refs(seed_blocks[-1]) == 0
    # every table page outside the prefix is the sequence's own
    own = st["block_table"][:, len(whole):]
    assert len(np.unique(own)) == own.size
