"""mx_moe_forward_noalloc (the forward whose workspace is the library's own
device-resident scratch) against mx_moe_forward with a caller workspace: same
kernels, so outputs, ids and weights must be identical bit for bit, on two
calls in a row (the second with fewer tokens, so it reads scratch the first
left behind), with and without an in-place residual."""
import ctypes as C

import numpy as np
import pytest
import torch

from maxuna_amd import ops
from maxuna_amd._lib import lib
from maxuna_amd.gguf import GgmlDType
from maxuna_amd.synth import CONFIGS, LayerSpec, build_layer, make_x
from tests.gpu_util import dev_f32, host

pytestmark = pytest.mark.gpu
MX_ERR_SCRATCH = 6


def test_noalloc_forward_matches_workspace_forward(dev):
    spec = CONFIGS["C2"]["spec"]
    layer = build_layer(spec, seed=1303, rms=True)
    blk = layer.block
    for t, seed in ((16, 1), (3, 2), (1, 3)):
        print(f"no-alloc t={t}", flush=True)
        x = dev_f32(make_x(spec, 500 + seed, t))
        want, wid, ww = blk.forward(x, return_routing=True)
        got, gid, gw = blk.forward_noalloc(x, return_routing=True)
        assert np.array_equal(host(got).view(np.uint32), host(want).view(np.uint32)), f"t={t}: out"
        assert np.array_equal(host(gid), host(wid)), f"t={t}: ids"
        assert np.array_equal(host(gw).view(np.uint32), host(ww).view(np.uint32)), f"t={t}: w"
        # in-place residual update, as the decoder chain uses it
        r1, r2 = x.clone(), x.clone()
        blk.forward(x, residual=r1, out=r1)
        blk.forward_noalloc(x, residual=r2, out=r2)
        assert np.array_equal(host(r1).view(np.uint32), host(r2).view(np.uint32)), f"t={t}: residual"


def test_noalloc_rejects_oversized_t(dev):
    spec = CONFIGS["C3"]["spec"]
    layer = build_layer(spec, seed=1304)
    assert lib().mx_moe_forward_noalloc_max_bytes() == 16 << 20
    x = dev_f32(make_x(spec, 600, 512))
    with pytest.raises(ops.MaxunaError, match="no-alloc forward: t = 512 needs"):
        layer.block.forward_noalloc(x)


def _largest_fitting_t(blk, cap):
    t = 1
    while lib().mx_moe_workspace_bytes(C.byref(blk._c), t + 1) <= cap:
        t += 1
    return t


def test_noalloc_grouped_path_and_limit(dev):
    """The f16 grouped paths from the static scratch.  C1 shape: t = 32 and the
    largest t whose workspace fits the 16 MiB scratch (57, as the header states)
    run the 16-pair MFMA tiles; a Q8_0 layer (hidden 1024, ff 512, 64 experts,
    top-4; a type the tiles do not take) runs the grouped GEMM (bucket map,
    GEMMs) at t = 32 and at its largest fitting t (510).  Each is bit-identical
    to the workspace forward, and t + 1 is rejected with MX_ERR_SCRATCH before
    any launch."""
    cap = lib().mx_moe_forward_noalloc_max_bytes()
    q8 = LayerSpec(1024, 512, 64, 4, GgmlDType.Q8_0, GgmlDType.Q8_0, shared=False)
    for spec, seed, want_max in ((CONFIGS["C2"]["spec"], 1307, 57), (q8, 1308, 510)):
        cfg = f"{spec.gate_dt.name}/{spec.hidden}"
        ts = (32,)
        blk = build_layer(spec, seed=seed).block
        t_max = _largest_fitting_t(blk, cap)
        assert t_max == want_max, (cfg, t_max)
        assert t_max >= ops.mm_id_min_seq()
        for t in ts + (t_max,):
            print(f"no-alloc grouped {cfg} t={t}", flush=True)
            x = dev_f32(make_x(spec, 900 + t, t))
            want, wid, ww = blk.forward(x, return_routing=True)
            got, gid, gw = blk.forward_noalloc(x, return_routing=True)
            assert np.array_equal(host(got).view(np.uint32), host(want).view(np.uint32)), f"t={t}: out"
            assert np.array_equal(host(gid), host(wid)), f"t={t}: ids"
            assert np.array_equal(host(gw).view(np.uint32), host(ww).view(np.uint32)), f"t={t}: w"
        x = dev_f32(make_x(spec, 999, t_max + 1))
        with pytest.raises(ops.MaxunaError) as ei:
            blk.forward_noalloc(x)
        assert ei.value.code == MX_ERR_SCRATCH, ei.value
