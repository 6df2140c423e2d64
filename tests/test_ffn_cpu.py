"""Host logic of the grouped NF4 expert FFN (no GPU): the reference wrapper's
argument checks (kernel/cpu_grouped.py:306-331), the device refusal, the
path choice and the sync-buffer size."""
import pytest
import torch

import _hiplib
import nf4_ffn


def _stack(E=4, H=64, K=128, n_dn=24):
    gu_p = torch.zeros(E, 2 * H, K // 2, dtype=torch.uint8)
    gu_a = torch.ones(E, 2 * H, K // 64)
    dn_p = torch.zeros(E, n_dn, H // 2, dtype=torch.uint8)
    dn_a = torch.ones(E, n_dn, H // 64)
    return gu_p, gu_a, dn_p, dn_a


def test_cpu_tensors_are_refused():
    gu_p, gu_a, dn_p, dn_a = _stack()
    with pytest.raises(RuntimeError) as ei:
        nf4_ffn.gemm_nf4_ffn_grouped(torch.zeros(3, 128, dtype=torch.bfloat16), gu_p, gu_a,
                                     dn_p, dn_a, [1, 2], [0, 3])
    assert "cuda" in str(ei.value).lower() and "dequant_ref" in str(ei.value)


def test_shape_checks_match_the_reference_messages():
    gu_p, gu_a, dn_p, dn_a = _stack()
    a = torch.zeros(3, 128, dtype=torch.bfloat16)
    chk = nf4_ffn._check
    assert chk(a, gu_p, gu_a, dn_p, dn_a, [1, 2], [0, 3]) == (3, 128, 64, 24)
    with pytest.raises(ValueError, match="even"):
        chk(a, gu_p[:, :-1], gu_a[:, :-1], dn_p, dn_a, [1, 2], [0, 3])
    with pytest.raises(ValueError, match="H % 64"):
        chk(a, gu_p[:, :64], gu_a[:, :64], dn_p, dn_a, [1, 2], [0, 3])
    with pytest.raises(ValueError, match="expert counts"):
        chk(a, gu_p, gu_a, dn_p[:2], dn_a[:2], [1, 2], [0, 3])
    with pytest.raises(ValueError, match="K mismatch"):
        chk(torch.zeros(3, 96, dtype=torch.bfloat16), gu_p, gu_a, dn_p, dn_a, [1, 2], [0, 3])
    with pytest.raises(AssertionError):
        chk(a, gu_p, gu_a, dn_p, dn_a, [1, 1], [0, 3])
    with pytest.raises(ValueError, match="group sizes"):
        chk(a, gu_p, gu_a, dn_p, dn_a, [1, 2], [0])
    with pytest.raises(TypeError):
        chk(a, gu_p, gu_a.double(), dn_p, dn_a, [1, 2], [0, 3])


def test_auto_path_threshold_in_units():
    # Qwen3 shapes: 48 gate/up + 64 down units per group
    assert nf4_ffn._fused_units(8, 768, 2048) == 8 * 112
    # batch 1 (8 groups) fuses; batch 2 (about 16 groups) composes
    assert nf4_ffn._fused_units(9, 768, 2048) <= nf4_ffn.FUSED_MAX_UNITS
    assert nf4_ffn._fused_units(10, 768, 2048) > nf4_ffn.FUSED_MAX_UNITS


def test_sync_words_follow_the_flag_layout():
    lib = _hiplib.load()
    assert lib.gnf4_hip_ffn_sync_words(8, 1536, 2048) == 16 + 8 * 64 * 48


def test_ffn_c_abi_rejects_bad_shapes_without_a_device():
    lib = _hiplib.load()
    base = dict(a=16, dt=0, lda=128, Bg=16, gsbe=8192, gsbn=64, Ag=16, gsae=256, gsan=2,
                Bd=16, dsbe=768, dsbn=32, Ad=16, dsae=24, dsan=1, eids=16, ro=16, G=2,
                max_m=2, N_gu=128, K=128, N_dn=24, h=16, ldh=64, sync=16, sync_words=4096,
                out=16, ldo=24, stream=None)

    def call(**over):
        args = dict(base)
        args.update(over)
        return lib.gnf4_hip_nf4_ffn_fwd(*args.values())

    assert call(N_gu=127) == -1            # odd gu width
    assert call(N_gu=96) == -1             # H % 64
    assert call(K=96) == -1
    assert call(max_m=17) == -1            # decode regime only
    assert call(ro=None) == -1             # row offsets needed above one row
    assert call(sync_words=8) == -1        # flags do not fit
    assert call(dt=1) == -1                # bf16 activations only
    assert call(ldh=60) == -1
    assert lib.gnf4_hip_silu_mul(16, 128, 4, 60, 16, 64, None) == -1    # H % 8
    assert lib.gnf4_hip_silu_mul(16, 100, 4, 64, 16, 64, None) == -1    # ldg < 2H
    assert lib.gnf4_hip_silu_mul(16, 128, 0, 64, 16, 64, None) == 0     # nothing to do
