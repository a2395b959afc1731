"""The gradient tolerance itself, on the CPU.

The GPU tests hold every gradient entry to rtol 1e-3 of the restatement's
plus that entry's own f32 rounding noise (tests/helpers.py: lane_noise,
propagate_noise); no tolerance is scaled by an array's largest entry.  This
file shows, at BASELINE.json's configs 0 and 1, that the tolerance

* admits a second, more accurate evaluation of the same gradient: the
  restatement's backward with every gradient quantity in double
  (oracle rasterize_backward_f64), for the lanes and, through project
  backward, for the dense gradients;
* rejects the plausible mistakes it exists to catch, planted in the
  restatement on the CPU:
  - the last batch of 64 entries of every tile's list dropped
    (OR_CHECK_DROP_LAST_BATCH);
  - the gradient rows of a third of the splats that have one set to zero
    (under a tolerance scaled by the array's largest entry about a third of
    such splats passed at config 1).
"""
import numpy as np
import pytest

from oracle import oracle as O
from brush_amd.camera import project_uniforms
from brush_amd.synthetic import CONFIGS, generate_splats, generate_v_output
from tests.helpers import OracleGrads, outside, propagate_noise

_cache = {}


def _case(k):
    if k not in _cache:
        _cache.clear()
        O.set_threads(O.max_threads())
        w = CONFIGS[k]
        tr, sh, op = generate_splats(w)
        vo = generate_v_output(w)
        u = project_uniforms(w.camera(), w.img_w, w.img_h, w.n, w.sh_degree)
        o = O.render_forward(u, tr, sh, op, O.FLAG_BWD_INFO)
        want = OracleGrads(o, tr, sh, op, vo, O.FLAG_REFINE_WEIGHT)
        _cache[k] = (tr, sh, op, vo, o, want)
    return _cache[k]


@pytest.mark.parametrize("k", [0, 1])
def test_tolerance_admits_the_float64_evaluation(k):
    tr, sh, op, vo, o, want = _case(k)
    v = o.num_visible
    exact = O.rasterize_backward_f64(o, vo, O.FLAG_REFINE_WEIGHT)
    bad, ratio = outside(exact[:v], want.v_combined[:v], want.lane_noise[:v])
    print(f"[tol] config {k} lanes, float64 evaluation: worst err/tol {ratio.max():.3g}")
    assert not bad.any()
    assert ratio.max() < 0.5, "less than 2x headroom for a correct evaluation"
    # the restatement itself is far from 1e-3 of the exact gradient in many
    # entries: the noise term is needed, not a convenience
    m = want.v_combined[:v, 0] != 0
    rel = np.abs(want.v_combined[:v, 0][m].astype(np.float64) - exact[:v, 0][m]) / np.abs(exact[:v, 0][m])
    print(f"[tol] config {k} lane 0: f32 vs float64 relative error median {np.median(rel):.2g} "
          f"p90 {np.quantile(rel, 0.9):.2g}")
    assert np.quantile(rel, 0.9) > 1e-4
    # dense gradients of the exact lanes
    dense = O.project_backward(o, tr, sh, op, exact)
    for name, got, w, n in (("v_transforms", dense[0], want.v_transforms, want.noise_transforms),
                            ("v_coeffs", dense[1], want.v_coeffs, want.noise_coeffs),
                            ("v_raw_opac", dense[2], want.v_raw_opac, want.noise_raw_opac)):
        bad, ratio = outside(got, w, n)
        print(f"[tol] config {k} {name}, float64 lanes: worst err/tol {ratio.max():.3g}")
        assert not bad.any()


@pytest.mark.parametrize("k", [0, 1])
def test_tolerance_rejects_a_dropped_last_batch(k):
    """Dropping the last batch of every tile's list moves the splats of those
    batches; each splat whose colour lanes (sums of vis v_out, well
    conditioned) move by more than 1 % must be rejected.  (A splat deep in
    one tile and shallow in others can move by less than rtol: no test at
    1e-3 can see that, and it is not counted.)"""
    tr, sh, op, vo, o, want = _case(k)
    v = o.num_visible
    planted, _, _ = O.rasterize_backward_check(o, vo, O.FLAG_REFINE_WEIGHT, check=O.CHECK_DROP_LAST_BATCH)
    bad, _ = outside(planted[:v], want.v_combined[:v], want.lane_noise[:v])
    w64 = want.v_combined[:v].astype(np.float64)
    moved = np.max(np.abs(planted[:v, 5:8] - w64[:, 5:8]) / np.maximum(np.abs(w64[:, 5:8]), 1e-38), axis=1) > 1e-2
    caught = np.any(bad, axis=1)
    print(f"[tol] config {k}: the dropped batches move {moved.sum()} rows by > 1 %; the tolerance rejects "
          f"{caught[moved].sum()} of them ({caught.sum()} rows rejected in all)")
    assert moved.sum() > 1000
    assert caught[moved].all()
    dense = O.project_backward(o, tr, sh, op, planted)
    bad_t, _ = outside(dense[0], want.v_transforms, want.noise_transforms)
    bad_c, _ = outside(dense[1], want.v_coeffs, want.noise_coeffs)
    rows = bad_t.any(1) | bad_c.reshape(bad_c.shape[0], -1).any(1)
    gfc = o.global_from_compact_gid.astype(np.int64)
    print(f"[tol] config {k}: dense rows of those splats rejected {rows[gfc[moved]].sum()} of {moved.sum()}")
    assert rows[gfc[moved]].all()


@pytest.mark.parametrize("k", [0, 1])
def test_tolerance_rejects_zeroed_gradient_rows(k):
    tr, sh, op, vo, o, want = _case(k)
    v = o.num_visible
    rows = np.nonzero(np.any(want.v_combined[:v] != 0, axis=1))[0]
    rng = np.random.default_rng(k)
    zero = rng.choice(rows, size=rows.size // 3, replace=False)
    planted = want.v_combined.copy()
    planted[zero] = 0.0
    bad, _ = outside(planted[:v], want.v_combined[:v], want.lane_noise[:v])
    caught = np.any(bad, axis=1)[zero]
    print(f"[tol] config {k}: {zero.size} of {rows.size} gradient rows zeroed, {caught.sum()} rejected")
    assert caught.all()
    # the same through the dense gradients (transforms and SH rows)
    gfc = o.global_from_compact_gid.astype(np.int64)
    dense = O.project_backward(o, tr, sh, op, planted)
    bad_t, _ = outside(dense[0], want.v_transforms, want.noise_transforms)
    bad_c, _ = outside(dense[1], want.v_coeffs, want.noise_coeffs)
    drow = bad_t.any(1) | bad_c.reshape(bad_c.shape[0], -1).any(1)
    print(f"[tol] config {k}: dense rows of zeroed splats rejected {drow[gfc[zero]].sum()} of {zero.size}")
    assert drow[gfc[zero]].all()


def test_noise_propagation_is_first_order_in_the_lanes():
    """propagate_noise is zero for zero lane noise and grows with it."""
    tr, sh, op, vo, o, want = _case(0)
    z = propagate_noise(o, tr, sh, op, want.v_combined, np.zeros_like(want.lane_noise), draws=1)
    assert all(not x.any() for x in z)
    small = propagate_noise(o, tr, sh, op, want.v_combined, want.lane_noise, draws=0)
    big = propagate_noise(o, tr, sh, op, want.v_combined, 8.0 * want.lane_noise, draws=0)
    assert big[0].sum() > 4.0 * small[0].sum()
