"""CPU check of the random-shape GPU sweep (tests/test_gpu_random_shapes.py): planning only
(no launch), so that the sweep keeps exercising every MFMA kernel family as the planners
change."""
import my_own_cnn_amd as M
from tests.test_gpu_random_shapes import ALGOS, SHAPES


def test_the_sweep_reaches_every_family():
    auto, accepting = set(), set()
    for n, h, wd, c, k, r, s, conv in SHAPES:
        kw = dict(padding=(conv[0], conv[1]), stride=(conv[2], conv[3]), dilation=(conv[4], conv[5]), groups=conv[6])
        auto.add(M.plan(M.make_desc((n, h, wd, c), (k, r, s, c // conv[6]), **kw)))
        for algo in ALGOS:
            try:
                M.plan(M.make_desc((n, h, wd, c), (k, r, s, c // conv[6]), algo=algo, **kw))
                accepting.add(algo)
            except M.MiqError:
                pass
    assert {"band", "stream", "igemm"} <= auto, auto
    assert set(ALGOS) <= accepting, accepting
