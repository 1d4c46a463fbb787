"""The GQA-indexed KV oracle against the tiled-cache form it restates.

``kv_reference_gqa``/``kv_tolerance_gqa`` must reproduce
``native_ops.kv_reference``/``kv_tolerance`` on the tiled inputs
(``kv_gqa_inputs``, the reference's own GQA test form,
tests/test_pack_kv_attention.py:176-205): the members bit for bit (same fp32
operations per head), the fp64 reference to fp64 rounding. A wrong head
mapping (h % HKV instead of h // r) or a dropped new entry moves both by
O(1).
"""

import numpy as np
import pytest

from oracle.extensions import kv_gqa_inputs, kv_reference_gqa, kv_tolerance_gqa
from oracle.native_ops import kv_reference, kv_tolerance
from oracle.verify import _Case


def case(b, h, hkv, t, dh, seed):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((b, h, dh)) * 0.3).astype(np.float16)
    kc = rng.standard_normal((hkv, t, dh)).astype(np.float16)
    vc = rng.standard_normal((hkv, t, dh)).astype(np.float16)
    nk = (rng.standard_normal((b, hkv, dh)) * 0.3).astype(np.float16)
    nv = rng.standard_normal((b, hkv, dh)).astype(np.float16)
    return q, kc, vc, nk, nv


@pytest.mark.parametrize("b,h,hkv,t,dh,bits", [(1, 8, 2, 64, 64, 8), (2, 4, 4, 33, 128, 4),
                                               (1, 8, 1, 100, 64, 3)])
def test_gqa_form_equals_tiled_form(b, h, hkv, t, dh, bits):
    q, kc, vc, nk, nv = case(b, h, hkv, t, dh, seed=t)
    tiled = kv_gqa_inputs(q, kc, vc, nk, nv, bits)
    ref_t = kv_reference(tiled)
    ref_g = kv_reference_gqa(q, kc, vc, nk, nv, bits)
    assert np.allclose(ref_g, ref_t, rtol=1e-12, atol=1e-14)
    for dtype in ("float16", "float32"):
        tol_t = kv_tolerance(_Case(dtype), tiled, ref_t)
        tol_g = kv_tolerance_gqa(dtype, q, kc, vc, nk, nv, bits, ref_t)
        assert tol_g == pytest.approx(tol_t, rel=1e-9), dtype


def test_wrong_head_mapping_is_caught():
    """Planted mistake: mapping h -> h % HKV must move the reference."""
    q, kc, vc, nk, nv = case(1, 8, 2, 64, 64, seed=1)
    good = kv_reference_gqa(q, kc, vc, nk, nv, 8)
    perm = np.arange(8).reshape(2, 4).T.reshape(-1)  # interleave heads as h % 2 would
    bad = kv_reference_gqa(q[:, perm], kc, vc, nk, nv, 8)[:, np.argsort(perm)]
    assert np.max(np.abs(good - bad)) > 1e-2
