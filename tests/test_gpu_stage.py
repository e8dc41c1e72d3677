"""A TRELLIS2 decoder stage loaded from a checkpoint-layout safetensors file
and run on the GPU (§ the reference's SparseStructuredLatentDecoder::
from_safetensors, sparse_decoder_runtime_impl.rs:94-190, and its stage
forward :522-1171).

The file holds stage 0 of a decoder at config 2's shape: model_channels
256 -> 128, two ConvNeXt blocks ``blocks.0.{0,1}.{conv, norm, mlp.0, mlp.2}``
(hidden width 1024, read from the file as load_linear_dynamic does) and the
upsample ``blocks.0.2.{norm1, to_subdiv, conv1, conv2}``; conv weights bf16,
the rest f32, as a TRELLIS2 checkpoint stores them.

* Both loaders -- ``bevy_synth_amd.loading`` and the C++ header through
  tests/cpp/test_loader -- put the same bits on the device, and those bits are
  the file's values in the compute dtype (bf16 RNE; f16-rounded biases and
  to_subdiv weights in f16 mode, the reference's bias_fp16 / weight_fp16).
* The stage on the config-2 shell (113,857 voxels): each ConvNeXt block at
  sampled rows against the oracle chain; the to_subdiv logits against the
  fp64 dense product; the children chosen by logit > 0
  (decoder_subdivision_child_thresholds with the default config) and their
  coords exactly against the oracle's subdivide_expand; the upsample's output
  at sampled children against the oracle chain of the fused C2S block.
* The reference's refusals: a missing key, a to_subdiv head of the wrong
  width, a conv1 of the wrong width -- same messages from both loaders.
"""
import os
import subprocess

import numpy as np
import pytest
import torch

from bevy_synth_amd import decoder as D
from bevy_synth_amd import loading as Ld
from bevy_synth_amd import synth
from tests.c2s_check import check_up_fused
from tests.sampling import sample_rows
from tests.test_loader import _bf16_bits, write_safetensors
from tests.tolerance import TOL_BF16, assert_close

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "test_loader")
C, C2, H, NB = 256, 128, 1024, 2


def stage_tensors(rng):
    """name -> (dtype, shape, f32 values as the file's dtype decodes them)."""
    T = {}

    def bf16(name, a):
        b = _bf16_bits(a)
        T[name] = ("BF16", a.shape, (b.astype(np.uint32) << 16).view(np.float32).reshape(a.shape), b.tobytes())

    def f32(name, a):
        a = np.asarray(a, np.float32)
        T[name] = ("F32", a.shape, a, a.tobytes())
    for b in range(NB):
        p = f"blocks.0.{b}"
        bf16(f"{p}.conv.weight", synth.normal_f32(rng, (C, 3, 3, 3, C), 1 / np.sqrt(27 * C)))
        f32(f"{p}.conv.bias", synth.normal_f32(rng, C, 0.1))
        f32(f"{p}.norm.weight", 1 + 0.1 * rng.standard_normal(C))
        f32(f"{p}.norm.bias", 0.1 * rng.standard_normal(C))
        bf16(f"{p}.mlp.0.weight", synth.normal_f32(rng, (H, C), 1 / np.sqrt(C)))
        f32(f"{p}.mlp.0.bias", synth.normal_f32(rng, H, 0.1))
        bf16(f"{p}.mlp.2.weight", synth.normal_f32(rng, (C, H), 1 / np.sqrt(H)))
        f32(f"{p}.mlp.2.bias", synth.normal_f32(rng, C, 0.1))
    p = f"blocks.0.{NB}"
    f32(f"{p}.norm1.weight", 1 + 0.1 * rng.standard_normal(C))
    f32(f"{p}.norm1.bias", 0.1 * rng.standard_normal(C))
    f32(f"{p}.to_subdiv.weight", synth.normal_f32(rng, (8, C), 1 / np.sqrt(C)))
    f32(f"{p}.to_subdiv.bias", synth.normal_f32(rng, 8, 0.2))
    bf16(f"{p}.conv1.weight", synth.normal_f32(rng, (8 * C2, 3, 3, 3, C), 1 / np.sqrt(27 * C)))
    f32(f"{p}.conv1.bias", synth.normal_f32(rng, 8 * C2, 0.1))
    bf16(f"{p}.conv2.weight", synth.normal_f32(rng, (C2, 3, 3, 3, C2), 1 / np.sqrt(27 * C2)))
    f32(f"{p}.conv2.bias", synth.normal_f32(rng, C2, 0.1))
    return T


def write(path, T, drop=(), replace=None):
    out = {k: (v[0], v[1], v[3]) for k, v in T.items() if k not in drop}
    out.update(replace or {})
    write_safetensors(str(path), out)


@pytest.fixture(scope="module")
def stage_file(tmp_path_factory):
    d = tmp_path_factory.mktemp("stage")
    T = stage_tensors(np.random.default_rng(2048))
    write(d / "stage.safetensors", T)
    return d, T


def run_cpp(path, outdir, dtype="bf16"):
    if not os.path.exists(BIN):
        pytest.skip("tests/cpp/test_loader is built by __graft_entry__.build()")
    os.makedirs(outdir, exist_ok=True)
    r = subprocess.run([BIN, "stage", str(path), str(outdir), "0", str(NB), str(C), str(C2), dtype],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    return dict(line.split(": ", 1) for line in open(os.path.join(outdir, "errors.txt")).read().splitlines())


def stage_device_tensors(stage):
    """checkpoint key -> the device tensor the Python-loaded stage holds."""
    out = {}
    for b, blk in enumerate(stage.convnext_blocks):
        p = f"blocks.0.{b}"
        out[f"{p}.conv.weight"], out[f"{p}.conv.bias"] = blk.conv.weight, blk.conv.bias
        out[f"{p}.norm.weight"], out[f"{p}.norm.bias"] = blk.norm_weight, blk.norm_bias
        out[f"{p}.mlp.0.weight"], out[f"{p}.mlp.0.bias"] = blk.mlp_0.weight, blk.mlp_0.bias
        out[f"{p}.mlp.2.weight"], out[f"{p}.mlp.2.bias"] = blk.mlp_2.weight, blk.mlp_2.bias
    u, p = stage.upsample, f"blocks.0.{NB}"
    out[f"{p}.norm1.weight"], out[f"{p}.norm1.bias"] = u.norm1_weight, u.norm1_bias
    out[f"{p}.to_subdiv.weight"], out[f"{p}.to_subdiv.bias"] = u.to_subdiv_weight, u.to_subdiv_bias
    out[f"{p}.conv1.weight"], out[f"{p}.conv1.bias"] = u.conv1.weight, u.conv1.bias
    out[f"{p}.conv2.weight"], out[f"{p}.conv2.bias"] = u.conv2.weight, u.conv2.bias
    return out


def raw_bytes(t):
    return t.contiguous().view(torch.uint8).cpu().numpy().tobytes()


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_stage_loaders_agree_with_the_file(oracle, stage_file, tmp_path, dtype):
    """Both loaders hold the same device bits, equal to the file's values in
    the compute dtype; the packed conv weights match between them."""
    d, T = stage_file
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    st = Ld.SafeTensors.open(str(d / "stage.safetensors"))
    stage = Ld.load_decoder_stage(st, 0, NB, C, C2, dtype=tdt)
    assert len(stage.convnext_blocks) == NB and stage.upsample is not None
    assert stage.upsample.compute_fp16 == (dtype == "f16")
    assert stage.convnext_blocks[0].mlp_0.weight.shape == (H, C)       # width from the file
    errs = run_cpp(d / "stage.safetensors", tmp_path / "cpp", dtype)
    assert errs == {}
    rnd = oracle.bf16_round if dtype == "bf16" else oracle.f16_round
    for key, t in stage_device_tensors(stage).items():
        got = raw_bytes(t)
        assert got == open(tmp_path / "cpp" / f"stage.{key}.bin", "rb").read(), key
        vals = T[key][2]
        f32_operand = key.endswith(".bias") or "to_subdiv" in key or ".norm" in key
        if f32_operand:
            exp = vals if (dtype == "bf16" or ".norm" in key) else oracle.f16_round(vals)
            assert t.dtype == torch.float32
            assert np.array_equal(t.cpu().numpy().ravel().view(np.uint32),
                                  np.asarray(exp, np.float32).ravel().view(np.uint32)), key
        else:
            assert t.dtype == tdt
            exp = rnd(vals).ravel()
            assert np.array_equal(t.float().cpu().numpy().ravel().view(np.uint32), exp.view(np.uint32)), key
    for b in range(NB + 1):
        for name in (["conv"] if b < NB else ["conv1", "conv2"]):
            layer = stage.convnext_blocks[b].conv if b < NB else getattr(stage.upsample, name)
            key = f"blocks.0.{b}.{name}"
            got = raw_bytes(layer.packed_weight())
            ref = open(tmp_path / "cpp" / f"stage.{key}.packed.bin", "rb").read()
            # the header's fields (magic .. bytes: 40 bytes; its padding is
            # never written) and the fragments after the 256-byte header
            assert got[:40] == ref[:40] and got[256:] == ref[256:], key


def _dense_f64(oracle, w, b, x):
    cout, cin = w.shape
    ident = np.arange(len(x), dtype=np.int32).reshape(-1, 1)
    return oracle.conv_gemm_f64(oracle.OracleConfig(cin, cout, 1, 1, 1), w.reshape(cout, 1, cin), b, x, ident)


def test_stage_forward_config2(oracle, stage_file):
    """The loaded stage on the config-2 shell: ConvNeXt x 2, then the C2S
    upsample whose children the to_subdiv logits choose."""
    d, T = stage_file
    r = oracle.bf16_round
    st = Ld.SafeTensors.open(str(d / "stage.safetensors"))
    stage = Ld.load_decoder_stage(st, 0, NB, C, C2, dtype=torch.bfloat16)
    coords = synth.config2_coords()
    rng = np.random.default_rng(99)
    x0 = r(synth.normal_f32(rng, (len(coords), C)))
    xd = torch.from_numpy(x0).cuda().to(torch.bfloat16)
    nb = D.Neighborhood.build(stage.convnext_blocks[0].conv.cfg, torch.from_numpy(coords).cuda())
    trace = []
    child_nb, y = stage.forward(nb, xd, trace=trace)
    kinds = [t[0] for t in trace]
    assert kinds == ["convnext", "convnext", "logits", "up"]

    # ConvNeXt blocks at sampled rows: conv -> LN(norm) -> mlp.0 -> SiLU -> mlp.2 + x
    rows = sample_rows(len(coords), rng, 1500, plan=nb.plan)
    m = nb.nbr.cpu().numpy()[rows]
    for _, b, xin, xout in trace[:2]:
        p = f"blocks.0.{b}"
        xi = xin.float().cpu().numpy()
        conv = oracle.conv_gemm_f64(oracle.OracleConfig(C, C), T[f"{p}.conv.weight"][2].reshape(C, 27, C),
                                    T[f"{p}.conv.bias"][2], xi, m).astype(np.float32)
        h = r(oracle.layer_norm(conv, T[f"{p}.norm.weight"][2], T[f"{p}.norm.bias"][2], 1e-6))
        hid = r(oracle.silu(_dense_f64(oracle, T[f"{p}.mlp.0.weight"][2], T[f"{p}.mlp.0.bias"][2], h)
                            .astype(np.float32)))
        exp = _dense_f64(oracle, T[f"{p}.mlp.2.weight"][2], T[f"{p}.mlp.2.bias"][2], hid) + xi[rows]
        assert_close(xout.float().cpu().numpy()[rows], exp, TOL_BF16, f"stage convnext block {b}")

    # to_subdiv logits (f32 skinny linear) against the fp64 product
    _, xp, logits = trace[2]
    xp_h = xp.float().cpu().numpy()
    lg = logits.cpu().numpy()
    p = f"blocks.0.{NB}"
    exp_lg = _dense_f64(oracle, T[f"{p}.to_subdiv.weight"][2], T[f"{p}.to_subdiv.bias"][2], xp_h)
    assert np.max(np.abs(lg - exp_lg)) <= 1e-4 * max(1.0, float(np.abs(exp_lg).max()))
    # children: logit > 0 (the default thresholds); where the fp64 logit is
    # farther than the f32 error from 0 the decision is the oracle's
    mask = lg > 0
    firm = np.abs(exp_lg) > 1e-4
    assert np.array_equal(mask[firm], (exp_lg > 0)[firm])
    # logits_to_mask + argwhere (the oracle's restatement) on the device logits
    pairs = oracle.subdivision_active(lg, np.array(D.DEFAULT_SUBDIVISION_THRESHOLDS, np.float32))
    assert np.array_equal(pairs, np.argwhere(mask))
    assert 0 < len(pairs) < 8 * len(coords)
    exp_cc, _ = oracle.subdivide_expand(coords, pairs)
    assert np.array_equal(child_nb.coords.cpu().numpy().astype(np.int64), exp_cc.astype(np.int64))
    assert tuple(y.shape) == (len(pairs), C2) and y.dtype == torch.bfloat16

    # the upsample at sampled children against the oracle chain
    crow = sample_rows(len(pairs), rng, 1500, plan=child_nb.plan)
    check_up_fused(oracle, stage.upsample, nb, xp, y, child_nb, pairs, crow)


@pytest.mark.parametrize("case,message", [
    ("missing", "missing tensor 'blocks.0.1.mlp.2.bias' in safetensors"),
    ("to_subdiv", "tensor 'blocks.0.2.to_subdiv.weight' expected out_channels=8, got 7"),
    ("conv1", "tensor 'blocks.0.2.conv1.weight' expected out_channels=1024, got 512"),
    ("norm", "tensor 'blocks.0.0.norm.weight' expected len=256, got len=255"),
])
def test_stage_refusals(stage_file, tmp_path, case, message):
    """The reference's checks, in its load order, with its messages, from both loaders."""
    d, T = stage_file
    p = f"blocks.0.{NB}"
    if case == "missing":
        write(tmp_path / "bad.safetensors", T, drop=("blocks.0.1.mlp.2.bias",))
    elif case == "to_subdiv":
        w = np.zeros((7, C), np.float32)
        write(tmp_path / "bad.safetensors", T, replace={f"{p}.to_subdiv.weight": ("F32", w.shape, w.tobytes())})
    elif case == "conv1":
        w = np.zeros((512, 3, 3, 3, C), np.float32)
        write(tmp_path / "bad.safetensors", T, replace={f"{p}.conv1.weight": ("F32", w.shape, w.tobytes())})
    else:
        w = np.ones(255, np.float32)
        write(tmp_path / "bad.safetensors", T, replace={"blocks.0.0.norm.weight": ("F32", w.shape, w.tobytes())})
    st = Ld.SafeTensors.open(str(tmp_path / "bad.safetensors"))
    with pytest.raises(Ld.LoadError) as e:
        Ld.load_decoder_stage(st, 0, NB, C, C2)
    assert str(e.value) == message
    assert run_cpp(tmp_path / "bad.safetensors", tmp_path / "cpp") == {"stage": message}
