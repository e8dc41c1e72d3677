"""The exact step bench.py times (config 3: 1,040,679 voxels, C = 128, bf16):
neighbour map -> conv plan -> conv3x3x3 -> LayerNorm -> SiLU (fused) ->
conv3x3x3 -> + x (fused), run through bench.Config3Step and checked against
the oracle chain at 3,000+ sampled output rows (the first and last tiles of
the plan's order included), after several back-to-back steps.  The map is
checked exactly against the oracle's at the sampled rows and their
neighbours."""
import numpy as np
import pytest
import torch

from tests.sampling import sample_rows
from tests.tolerance import TOL_BF16, assert_close

pytestmark = pytest.mark.gpu


def test_config3_bench_step_matches_oracle(oracle):
    import bench

    st = bench.Config3Step(torch.device("cuda:0"))
    for _ in range(3):  # the bench's steps rebuild the map and plan each time
        st.step()
    st.F.neighbor_map_check(st.ws)
    torch.cuda.synchronize()
    n, C = st.n, st.C
    rng = np.random.default_rng(33)
    rows = sample_rows(n, rng, 3000, plan=st.plan)
    assert len(rows) >= 3000
    nbr = st.nbr.cpu().numpy()
    ocfg = oracle.OracleConfig(C, C)
    # the map at the sampled rows and at the rows conv2 reads, exactly
    r1 = np.unique(nbr[rows][nbr[rows] >= 0])
    chk = np.unique(np.concatenate([rows, r1]))
    exp_map = oracle.build_neighbor_rows(ocfg, st.coords)
    assert np.array_equal(nbr[chk], exp_map[chk])
    # conv1 -> LN -> SiLU (rounded to bf16, as h is stored) at r1, then conv2 + x
    b = np.zeros(C, np.float32)
    n1 = nbr[r1]
    h1 = oracle.conv_gemm_f64(ocfg, st.w1, b, st.x_f32, n1)
    h = oracle.bf16_round(oracle.silu(oracle.layer_norm(h1.astype(np.float32), None, None, 1e-6)))
    # h at the device's h rows r1, zeros elsewhere (conv2 at `rows` reads only r1)
    loc = np.where(nbr[rows] >= 0, np.searchsorted(r1, np.maximum(nbr[rows], 0)), -1)
    y = oracle.conv_gemm_f64(ocfg, st.w2, b, h, loc) + st.x_f32[rows]
    got = st.out.float().cpu().numpy()[rows]
    assert_close(got, y, TOL_BF16, "config 3 bench step")
    # the intermediate h as stored by conv1's fused epilogue
    assert_close(st.h.float().cpu().numpy()[r1], h, TOL_BF16, "config 3 conv1 -> LN -> SiLU")
