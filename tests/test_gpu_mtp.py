"""GPU parity: draft-pass metadata (pkv_mtp_next, and the reference-named
mtp_next of pkv_kernels.hsaco launched as the reference does) against the
oracle (oracle/pkv_oracle.c orc_mtp_next, restating qwen35.cu:2633-2650).
Integer work: bit-exact."""
import numpy as np
import pytest
import torch

import oracle
import pkv
from _util import BS
from pkv.refabi import I, P, RefKernels

pytestmark = pytest.mark.gpu


def case(S, seed):
    rng = np.random.default_rng(seed)
    max_blocks = 12
    T = 3 * S
    rows = np.sort(rng.choice(T, S, replace=False)).astype(np.int32)  # one step row per sequence
    pos = rng.integers(0, max_blocks * BS - 8, T).astype(np.int32)
    bt = rng.permutation(S * max_blocks).reshape(S, max_blocks).astype(np.int32)
    # limits: the last position each sequence holds, some below the draft position (-> -1), padding -1
    limits = (pos[rows] + rng.integers(-2, 6, S)).astype(np.int32)
    limits[::5] = -1
    rope_stride = T + 3
    rope = rng.integers(0, 1 << 20, 3 * rope_stride).astype(np.int32)
    return dict(rows=rows, pos=pos, rope=rope, rope_stride=rope_stride, bt=bt, max_blocks=max_blocks, limits=limits,
                S=S)


def dev32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)


@pytest.mark.parametrize("S,k,seed,refabi", [(1, 1, 0, False), (37, 2, 1, False), (300, 3, 2, False),
                                             (37, 1, 3, True), (300, 4, 4, True)])
def test_mtp_next_matches_oracle(dev, S, k, seed, refabi):
    print(f"case mtp_next S={S} k={k} refabi={refabi}", flush=True)
    c = case(S, seed)
    want = oracle.mtp_next(c["rows"], c["pos"], c["rope"], c["rope_stride"], c["bt"], c["max_blocks"], BS,
                           c["limits"], k)
    args = [dev32(c[n], dev) for n in ("rows", "pos", "rope")]
    bt, lim = dev32(c["bt"], dev), dev32(c["limits"], dev)
    dpos = torch.full((S,), -7, dtype=torch.int32, device=dev)
    dslot = torch.full((S,), -7, dtype=torch.int32, device=dev)
    drope = torch.full((3, S), -7, dtype=torch.int32, device=dev)
    if refabi:
        RefKernels().launch("mtp_next", ((S + 127) // 128, 1, 1), 128, 0,
                            [P(args[0]), P(args[1]), P(args[2]), I(c["rope_stride"]), P(bt), I(c["max_blocks"]),
                             I(BS), P(lim), I(k), P(dpos), P(dslot), P(drope), I(S)])
    else:
        pkv.mtp_next(*args, c["rope_stride"], bt, c["max_blocks"], BS, lim, k, dpos, dslot, drope, S)
    torch.cuda.synchronize()
    assert np.array_equal(dpos.cpu().numpy(), want[0])
    assert np.array_equal(dslot.cpu().numpy(), want[1])
    assert np.array_equal(drope.cpu().numpy(), want[2])
    if S > 5:  # both branches of the limit covered
        assert (want[1] == -1).any() and (want[1] >= 0).any()
