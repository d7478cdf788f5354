"""GGUF ingestion on the GPU: a synthetic layer exported with the reference's
tensor names, read back through the native reader into HBM (pinned staging,
chunked DMA) and run through the MoE block.  Expected: byte-identical expert
stacks and an output bit-identical to the layer built in memory (same bytes,
same kernels), plus the oracle check on the loaded layer."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from maxuna_amd import gguf as G
from maxuna_amd.loader import export_layer, load_moe_block
from maxuna_amd.synth import CONFIGS, build_layer, make_x
from tests.gpu_util import assert_close, dev_f32, host

pytestmark = pytest.mark.gpu


def test_gguf_layer_roundtrip(dev, orc, tmp_path):
    print("gguf C0 roundtrip", flush=True)
    spec = CONFIGS["C0"]["spec"]
    layers = [build_layer(spec, seed=77, layer=i) for i in range(2)]
    path = tmp_path / "c0.gguf"
    export_layer(path, layers)
    with G.GgufFile(path) as gf:
        assert gf.get_int("laguna.expert_count") == spec.n_expert
        for li, lay in enumerate(layers):
            blk = load_moe_block(gf, li, with_norm=False)
            for mine, theirs in ((blk.experts.gate, lay.block.experts.gate),
                                 (blk.experts.down, lay.block.experts.down)):
                assert (mine.dtype, mine.n_expert, mine.n_out, mine.k) == \
                    (theirs.dtype, theirs.n_expert, theirs.n_out, theirs.k)
                assert torch.equal(mine.buffer[:mine.nbytes].cpu(), theirs.buffer[:theirs.nbytes].cpu())
            assert blk.cfg.n_expert_used == spec.top_k
            x = make_x(spec, 5, 3, layer=li)
            out_l, ids_l, w_l = blk.forward(dev_f32(x), return_routing=True)
            out_m, ids_m, w_m = lay.block.forward(dev_f32(x), return_routing=True)
            assert np.array_equal(host(ids_l), host(ids_m))
            assert np.array_equal(host(out_l), host(out_m))  # same bytes, same kernels
            want, _, _ = orc.moe_layer(spec, lay.keys, lay.router_t, lay.bias, x, ids=host(ids_l), w=host(w_l))
            assert_close(host(out_l), want, what=f"gguf layer {li}")


def test_gguf_chunked_upload(dev, tmp_path):
    """A tensor larger than the 32 MiB staging chunk (double-buffered path)."""
    print("gguf chunked upload", flush=True)
    rng = np.random.default_rng(3)
    big = rng.integers(0, 256, 80 * 2**20 + 144 * 7, dtype=np.uint8)  # 80 MiB + a ragged tail
    n_blocks = big.size // 144
    raw = big[:n_blocks * 144]
    path = tmp_path / "big.gguf"
    G.write_gguf(path, {}, [("small", 0, (3,), np.float32([1, 2, 3]).tobytes()),
                            ("big", 12, (n_blocks, 256), raw.tobytes())], alignment=64)
    with G.GgufFile(path) as gf:
        got = gf.read_device("big")
        assert torch.equal(got.cpu(), torch.from_numpy(raw))
        assert torch.equal(gf.dense_f32("small").cpu(), torch.tensor([1.0, 2.0, 3.0]))
