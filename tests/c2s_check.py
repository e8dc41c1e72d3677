"""Oracle chain of the fused C2S upsample block at sampled children, shared by
the C2S and decoder GPU tests."""
import numpy as np
import torch

from tests.tolerance import TOL_BF16, assert_close


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.float().cpu().numpy()


def check_up_fused(oracle, up, parent_nb, x_dev, y_dev, child_nb, pairs, rows, w_scale=True):
    """The fused C2SUpsampleBlock at sampled children against the oracle chain:
    SiLU(LN(x; norm1)) (bf16) -> conv1 (f32, not rounded) -> child slice ->
    SiLU(LN) (bf16) -> conv2 -> + channel-repeated parent skip -> bf16."""
    r = oracle.bf16_round
    cin, cout = up.in_channels, up.out_channels
    li = pairs[:, 0] * 8 + pairs[:, 1]
    nc = child_nb.nbr[dev(rows.astype(np.int64))].cpu().numpy()
    rc = np.unique(nc[nc >= 0])                          # children whose h_up conv2 reads
    par = np.unique(li[rc] // 8)                         # their parents (conv1 rows)
    npar = parent_nb.nbr[dev(par.astype(np.int64))].cpu().numpy()
    rp = np.unique(npar[npar >= 0])                      # the parents conv1 reads
    n1w, n1b = up.norm1_weight.cpu().numpy(), up.norm1_bias.cpu().numpy()
    h0 = r(oracle.silu(oracle.layer_norm(host(x_dev[dev(rp.astype(np.int64))]), n1w, n1b, 1e-6)))
    loc = np.where(npar >= 0, np.searchsorted(rp, np.maximum(npar, 0)), -1)

    def weights(layer):
        q = layer.weight.cpu()
        wf = q.float().numpy() if q.dtype != torch.bfloat16 else host(q)
        return wf, (layer.w_scale.cpu().numpy() if layer.w_scale is not None else None)
    w1, s1 = weights(up.conv1)
    h1 = oracle.conv_gemm_f64(oracle.OracleConfig(cin, 8 * cout), w1, up.conv1.bias.cpu().numpy(), h0, loc, s1)
    sl = h1.reshape(len(par), 8, cout)[np.searchsorted(par, li[rc] // 8), li[rc] % 8].astype(np.float32)
    hup = r(oracle.silu(oracle.layer_norm(sl, None, None, 1e-6)))
    loc2 = np.where(nc >= 0, np.searchsorted(rc, np.maximum(nc, 0)), -1)
    w2, s2 = weights(up.conv2)
    y = oracle.conv_gemm_f64(oracle.OracleConfig(cout, cout), w2, up.conv2.bias.cpu().numpy(), hup, loc2, s2)
    pf = host(x_dev[dev((li[rows] // 8).astype(np.int64))]).reshape(len(rows), 8, cin // 8)
    skip = pf[np.arange(len(rows)), li[rows] % 8]
    y = y + np.repeat(skip, cout // (cin // 8), axis=1)
    assert_close(host(y_dev[dev(rows.astype(np.int64))]), y, TOL_BF16, "fused c2s upsample block")
