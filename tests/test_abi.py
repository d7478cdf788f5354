"""CPU-side checks of the C ABI: the library loads, exports every entry point the
header declares, and rejects malformed calls on the host with the documented
status code before touching the GPU (reference: dispatch.rs:812-847,
mv_id.rs:138 / mm_id.rs:380 `shape_mismatch_errors`)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from maxuna_amd import _lib
from maxuna_amd._lib import ExpertStackC, Map0C, MoeLayerC

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "maxuna_moe.h"
INSTRUMENT = ROOT / "maxuna_amd" / "csrc" / "mx_instrument.h"
FAKE = 0x10000  # an aligned address no test ever lets reach a launch


def declared_symbols(path=HEADER):
    text = path.read_text()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(mx_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    syms = declared_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(L, s), s
    assert set(syms) == set(_lib.SIGNATURES), set(syms) ^ set(_lib.SIGNATURES)


def test_instrumentation_stays_outside_the_boundary_header():
    """The bench-only hooks are exported but declared only in the internal
    instrumentation header, never in the boundary header."""
    L = _lib.lib()
    inst = declared_symbols(INSTRUMENT)
    assert set(inst) == set(_lib.INSTRUMENT_SIGNATURES), inst
    assert not set(inst) & set(declared_symbols())
    for s in inst:
        assert hasattr(L, s), s


def test_block_geometry():
    L = _lib.lib()
    assert (L.mx_block_size(12), L.mx_type_size(12)) == (256, 144)
    assert (L.mx_block_size(14), L.mx_type_size(14)) == (256, 210)
    assert (L.mx_block_size(8), L.mx_type_size(8)) == (32, 34)
    assert L.mx_block_size(2) == -1 and L.mx_type_size(99) == -1
    assert b"gfx950" in L.mx_version()


def stack(dtype=12, n_expert=4, n_out=8, k=256, base_off=0, data=FAKE):
    return ExpertStackC(data, base_off, dtype, 0, n_expert, n_out, k)


def mv(st, t=3, xpr=1, k=256, ids_t=3, top_k=2, x=FAKE, ids=FAKE, dst=FAKE):
    L = _lib.lib()
    return L.mx_mul_mv_id(C.byref(st), x, t, xpr, k, ids, ids_t, top_k, dst, None)


def err():
    return _lib.lib().mx_last_error().decode()


def test_mul_mv_id_validation():
    assert mv(stack(), k=512) == 2 and "does not match expert stack k" in err()
    assert mv(stack(), ids_t=4) == 2 and "ids t" in err()
    assert mv(stack(), xpr=3) == 5 and "x_per_row" in err()
    assert mv(stack(dtype=2)) == 3
    assert mv(stack(k=250), k=250) == 4 and "block size" in err()
    assert mv(stack(data=None)) == 1
    assert mv(stack(), x=None) == 1
    assert mv(stack(), dst=FAKE + 4) == 9
    assert mv(stack(base_off=4)) == 9          # Q4_K rows need 16-byte alignment
    assert mv(stack(), top_k=0) == 8
    assert mv(stack(), t=0, ids_t=0) == 0      # empty is a no-op, not an error
    # Q6_K/Q8_0 need 2-byte alignment only (t=0: validated, nothing launched)
    assert mv(stack(dtype=14, k=256, base_off=2), k=256, t=0, ids_t=0) == 0
    assert mv(stack(dtype=8, k=256, base_off=1), k=256) == 9
    assert mv(stack(n_expert=40000)) == 7


def test_mul_mm_id_shared_geometry_mismatch():
    L = _lib.lib()
    st = stack(n_expert=32, n_out=64)
    good = L.mx_map0_scratch_bytes(32, 48, 10)
    m = Map0C(FAKE, good, 32, 48, 10)
    for bad in (Map0C(FAKE, good, 31, 48, 10), Map0C(FAKE, good, 32, 47, 10), Map0C(FAKE, good, 32, 48, 9)):
        rc = L.mx_mul_mm_id_shared(C.byref(st), FAKE, 48, 1, 256, FAKE, 48, 10, C.byref(bad), FAKE, None)
        assert rc == 6 and "does not match this projection" in err()
    small = Map0C(FAKE, good - 4, 32, 48, 10)
    assert L.mx_mul_mm_id_shared(C.byref(st), FAKE, 48, 1, 256, FAKE, 48, 10, C.byref(small), FAKE, None) == 6
    # ids t disagreeing with x t (mm_id.rs:380-390)
    assert L.mx_mul_mm_id_shared(C.byref(st), FAKE, 16, 1, 256, FAKE, 8, 2, C.byref(m), FAKE, None) == 2


def test_map0_validation():
    L = _lib.lib()
    assert L.mx_prepare_map0(0, FAKE, 4, 2, FAKE, 1 << 20, None) == 2
    assert L.mx_prepare_map0(8, FAKE, 4, 9, FAKE, 1 << 20, None) == 8
    need = L.mx_map0_scratch_bytes(8, 4, 2)
    assert need > 0
    assert L.mx_prepare_map0(8, FAKE, 4, 2, FAKE, need - 1, None) == 6


def test_combine_guards():
    L = _lib.lib()
    # i32 index overflow guard (dispatch.rs:2187-2199)
    per_seq = 10 * 3072
    max_ok = (2**31 - 1) // per_seq
    assert L.mx_combine(FAKE, None, FAKE, max_ok + 1, 10, 3072, FAKE, None) == 7
    assert L.mx_combine(FAKE, None, FAKE, 3, 0, 3072, FAKE, None) == 2
    assert L.mx_combine(None, None, FAKE, 3, 10, 64, FAKE, None) == 1


def test_route_validation():
    L = _lib.lib()
    assert L.mx_route_from_logits(FAKE, FAKE, 1, 2048, 10, 1.0, 1, FAKE, FAKE, None) == 2
    assert L.mx_route_from_logits(FAKE, FAKE, 1, 8, 9, 1.0, 1, FAKE, FAKE, None) == 8
    assert L.mx_route_from_logits(FAKE, FAKE, 1, 64, 33, 1.0, 1, FAKE, FAKE, None) == 8


def _layer(**kw):
    H, FF, E = 256, 512, 8
    d = dict(router=FAKE, exp_probs_b=FAKE, gate=stack(12, E, FF, H), up=stack(12, E, FF, H),
             down=stack(14, E, H, FF), shared_gate=ExpertStackC(), shared_up=ExpertStackC(),
             shared_down=ExpertStackC(), hidden=H, expert_ff=FF, top_k=2, weights_scale=1.0,
             weights_norm=1, mm_min_seq=0, rms_alpha=None, rms_eps=1e-6, reserved=0)
    d.update(kw)
    return MoeLayerC(**d)


def test_moe_forward_validation():
    L = _lib.lib()
    run = lambda lay, t=1, ws=1 << 24: L.mx_moe_forward(C.byref(lay), FAKE, t, None, FAKE, None, None,  # noqa
                                                        FAKE, ws, None)
    assert run(_layer(up=stack(12, 7, 512, 256))) == 2 and "disagree on n_expert" in err()
    assert run(_layer(up=stack(14, 8, 512, 256))) == 3 and "share a quant type" in err()
    assert run(_layer(top_k=9)) == 8
    assert run(_layer(router=None)) == 1
    lay = _layer()
    need = L.mx_moe_workspace_bytes(C.byref(lay), 1)
    assert need > 0
    assert run(lay, ws=need - 1) == 6
    # the grouped path needs more workspace than decode
    assert L.mx_moe_workspace_bytes(C.byref(lay), 64) > need


def test_tensor_key_agrees_with_python():
    from maxuna_amd.synth import tensor_key
    L = _lib.lib()
    for args in [(0, 0, 0), (7, 3, 12), (2**40 + 3, 47, 22)]:
        assert L.mx_tensor_key(*args) == tensor_key(*args)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "nope.so")
    with pytest.raises(RuntimeError, match="no non-native fallback"):
        _lib.lib()
