"""CPU checks of tests/helpers.poison_unneeded, the cache poisoner the GPU
guard tests use: it must poison slots of every kind the call may not read
and none that it must read.  The FP64 oracle (which reads only the slots of
[begin, end) that some query row can see) is the judge: its output is bitwise
unchanged by the poisoning, and poisoning one needed slot changes it."""
import copy

import numpy as np

from kvbridge_amd import workloads as W
from oracle import oracle as O

from helpers import poison_unneeded


def _cases():
    yield W.synth_case(1, 8, 2, 64, 64, 1000, seed=5, pages=20, begin=37, end=950, qpos=[700])
    yield W.synth_case(1, 4, 1, 96, 48, 500, seed=6, begin=0, end=481, qpos=[10_000])
    yield W.synth_case(1, 4, 2, 64, 16, 300, seed=7, begin=10, end=290, qpos=[200], int8=False)
    f = O.fixture(513, permute=True)
    f.qpos = np.array([0, 33, 250, 255, 256, 400, 410, 420], np.int64)
    yield f


def test_poison_keeps_oracle_bitwise():
    for case in _cases():
        ref, vis = O.fp64(case)
        pc, nbad = poison_unneeded(case)
        assert nbad > 0
        out, vis2 = O.fp64(pc)
        assert np.array_equal(vis, vis2)
        assert np.array_equal(ref.view(np.uint64), out.view(np.uint64)), case.shape.as_tuple()


def test_poisoning_a_needed_slot_is_caught():
    # Planted mistake: one slot the call must read gets the poison too; the
    # oracle output must change, so the bitwise check above can fail.
    case = next(_cases())
    s = case.shape
    ref, _ = O.fp64(case)
    t = s.begin + 5  # visible: k_position 42 <= 700
    pc = copy.deepcopy(case)
    pg, sl = int(case.table[t // s.page_tokens]), t % s.page_tokens
    pc.k[pg, :, sl, :] = 127
    pc.v[pg, :, :, sl] = -128
    pc.ks[pg, :, sl] = 1.0e4
    pc.vs[pg, :, sl] = 1.0e4
    out, _ = O.fp64(pc)
    assert not np.array_equal(ref, out)


def test_poison_covers_every_kind():
    # tokens before begin, after the last visible position, past end in the
    # last page, and pool pages the range does not map: all poisoned.
    case = W.synth_case(1, 8, 2, 64, 64, 1000, seed=5, pages=20, begin=37, end=950, qpos=[700])
    s = case.shape
    pc, nbad = poison_unneeded(case)
    P = s.page_tokens
    poisoned = pc.ks[:, 0, :] == np.float32(1.0e4)
    for t in (0, 36, 701, 949, 950, 1023):
        assert poisoned[case.table[t // P], t % P], t
    for t in (37, 400, 700):
        assert not poisoned[case.table[t // P], t % P], t
    used = {int(case.table[lp]) for lp in range(-(-s.end // P))}
    for pg in set(range(s.pages)) - used:
        assert poisoned[pg].all()
    assert nbad == int(poisoned.sum())
