"""GPU parity at BASELINE.json's full sizes.

Configs 0 (100k SH0 splats at 256x256), 1 (the north-star workload, 1M SH3
splats at 1920x1080) and 2 (3M clustered splats, 93M tile intersections) are
compared with the CPU restatement bit for bit through the forward and to the
gradient tolerance through the backward, every splat.  All configs, and config
3 (6M splats at 3840x2160, forward only, all eight poses), are also checked
through properties that do not need the CPU run:

* the tile sort: tile ids non-decreasing, compact ids increasing inside each
  tile, every compact id appearing exactly as often as its splat's tile count,
  tile offsets equal to the runs;
* the depth sort: depths non-decreasing, global ids a permutation of the
  visible splats;
* per-splat outputs (tile count, max radius, projected row, the list of tiles
  a splat lands in) depend on the splat alone, so the CPU restatement run on a
  random subset of splats must reproduce them bit for bit;
* the image is finite with alpha in [0, 1]; gradients are finite.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import (OracleGrads, assert_bits_equal, check_fused_backward, compare_forward, gpu_forward,
                           keep_lanes, uniforms_for)
from brush_amd.synthetic import CONFIGS, generate_splats, generate_v_output  # noqa: F401

pytestmark = pytest.mark.gpu

_splats = {}


@pytest.fixture(autouse=True, scope="module")
def _oracle_threads():
    """The restatement runs these sizes on the box's CPU share (16 threads)."""
    import os

    O.set_threads(max(1, min(16, os.cpu_count() or 1)))
    yield
    O.set_threads(1)


def _scene(k):
    """The config's splats, generated once per test session."""
    if k not in _splats:
        _splats.clear()
        _splats[k] = generate_splats(CONFIGS[k])
    return _splats[k]


def _check_sort_structure(g, num_tiles):
    v, m = g["num_visible"], g["num_intersections"]
    tiles = g["tile_id_from_isect"].astype(np.int64)
    cg = g["compact_gid_from_isect"].astype(np.int64)
    assert tiles.shape == (m,) and cg.shape == (m,)
    assert m == 0 or tiles.max() < num_tiles, "sentinel or out-of-range tile id"
    d = np.diff(tiles)
    assert np.all(d >= 0), "tile ids not sorted"
    same = d == 0
    assert np.all(np.diff(cg)[same] > 0), "compact ids not increasing inside a tile"
    gfc = g["global_from_compact_gid"].astype(np.int64)
    counts = g["intersect_counts"].astype(np.int64)
    assert np.array_equal(np.bincount(cg, minlength=v)[:v], counts[gfc]), "per-splat entry counts"
    assert counts.sum() == m
    depths = g["depths"]
    assert np.all(np.diff(depths) >= 0), "depths not sorted"
    assert gfc.size == v and (v == 0 or gfc.max() < counts.size), "global ids out of range"
    assert np.unique(gfc).size == v, "global ids repeat"
    # tile offsets are the runs (empty tiles [0, 0])
    t = np.arange(num_tiles)
    start = np.searchsorted(tiles, t, "left")
    end = np.searchsorted(tiles, t, "right")
    empty = start == end
    start[empty] = 0
    end[empty] = 0
    pre = g["tile_offsets_pre"].reshape(-1, 2).astype(np.int64)
    assert np.array_equal(pre[:, 0], start) and np.array_equal(pre[:, 1], end), "tile offsets"
    post = g["tile_offsets"].reshape(-1, 2).astype(np.int64)
    assert np.array_equal(post[:, 0], start), "post-raster tile starts"
    assert np.all(post[:, 1] <= end) and np.all(post[:, 1] >= post[:, 0]), "post-raster tile ends"


def _check_subset(g, u, tr, sh, opac, flags, seed, size=20000):
    """Per-splat outputs of a random subset against the restatement run on that subset."""
    n = tr.shape[0]
    rng = np.random.default_rng(seed)
    sub = np.sort(rng.choice(n, size=min(size, n), replace=False))
    o = O.render_forward(u, tr[sub], sh[sub], opac[sub], flags)
    assert_bits_equal("subset intersect_counts", g["intersect_counts"][sub], o.intersect_counts)
    assert_bits_equal("subset max_radius", g["max_radius"][sub], o.max_radius)
    # projected rows: GPU row of global id x sits at its compact position
    gfc = g["global_from_compact_gid"].astype(np.int64)
    pos = np.full(n, -1, np.int64)
    pos[gfc] = np.arange(gfc.size)
    sub_vis = sub[o.global_from_compact_gid.astype(np.int64)]  # global ids, in the subset's depth order
    assert np.all(pos[sub_vis] >= 0), "a splat visible on its own is culled in the full scene"
    assert_bits_equal("subset projected rows", g["projected"][pos[sub_vis]], o.projected[: o.num_visible])
    # the tiles each subset splat lands in
    in_sub = np.zeros(n, bool)
    in_sub[sub] = True
    cg = g["compact_gid_from_isect"].astype(np.int64)
    gids = gfc[cg]
    keep = in_sub[gids]
    got = np.lexsort((g["tile_id_from_isect"][keep], gids[keep]))
    got_pairs = np.stack([gids[keep][got], g["tile_id_from_isect"][keep][got].astype(np.int64)], 1)
    m = o.num_intersections
    o_g = sub[o.global_from_compact_gid.astype(np.int64)[o.compact_gid_from_isect[:m].astype(np.int64)]]
    o_t = o.tile_id_from_isect[:m].astype(np.int64)
    ref = np.lexsort((o_t, o_g))
    ref_pairs = np.stack([o_g[ref], o_t[ref]], 1)
    assert np.array_equal(got_pairs, ref_pairs), "(splat, tile) pairs of the subset"


def _check_image(img):
    assert np.all(np.isfinite(img)), "non-finite pixels"
    a = img[..., 3]
    assert a.min() >= 0.0 and a.max() <= 1.0
    assert img[..., :3].min() >= 0.0


@pytest.mark.parametrize("w_id", [0, 1])
def test_full_size_forward_and_backward(gpu, w_id):
    """Configs 0 and 1 (the north-star workload) bit for bit (forward) and to
    rtol 1e-3 (gradients, every splat)."""
    import torch
    from brush_amd import render as R

    w = CONFIGS[w_id]
    print(f"[case] {w.name} forward + backward", flush=True)
    tr, sh, opac = _scene(w_id)
    cam = w.camera()
    u = uniforms_for(cam, w.img_w, w.img_h, w.n, w.sh_degree)
    g = gpu_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    o = O.render_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    compare_forward(g, o)
    _check_sort_structure(g, u["tile_bw"] * u["tile_bh"])
    del g
    _compare_gradients(gpu, w, cam, tr, sh, opac, o)


def _compare_gradients(gpu, w, cam, tr, sh, opac, o):
    """The fused backward of render_splats_diff against the restatement's
    rasterize + project backward for the config's upstream gradient: its
    per-splat lanes entry by entry, its dense gradients bit for bit against
    the restatement's project backward of those lanes, and entry by entry
    against the restatement's own dense gradients; every entry within rtol
    1e-3 plus its own f32 rounding noise (tests/helpers.py), with the worst
    err / tol printed per array."""
    import torch
    from brush_amd import render as R

    t = torch.from_numpy(tr).to(gpu).requires_grad_(True)
    s = torch.from_numpy(sh).to(gpu).requires_grad_(True)
    op = torch.from_numpy(opac).to(gpu).requires_grad_(True)
    v_out = generate_v_output(w)
    with keep_lanes():
        res = R.render_splats_diff(R.Splats(t, s, op), cam, (w.img_w, w.img_h))
        res.img.backward(torch.from_numpy(v_out).to(gpu))
    want = OracleGrads(o, tr, sh, opac, v_out, O.FLAG_REFINE_WEIGHT)
    grads = {"v_transforms": t.grad.cpu().numpy(), "v_coeffs": s.grad.cpu().numpy(),
             "v_raw_opac": op.grad.cpu().numpy(), "v_refine": res._cfg.refine_weight.cpu().numpy()}
    check_fused_backward(w.name, res._cfg.state, tr, sh, opac, grads, want)


def test_config2_clustered_full_size(gpu):
    """3M clustered splats at 1280x720: the high-overlap intersect / sort
    stress, against the restatement bit for bit (forward) and to rtol 1e-3
    (gradients, every splat)."""
    import gc

    w_id = 2
    w = CONFIGS[w_id]
    print(f"[case] {w.name} forward + backward", flush=True)
    tr, sh, opac = _scene(w_id)
    cam = w.camera()
    u = uniforms_for(cam, w.img_w, w.img_h, w.n, w.sh_degree)
    g = gpu_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    print(f"[case] {w.name}: visible={g['num_visible']} intersections={g['num_intersections']}", flush=True)
    assert g["num_intersections"] > 20_000_000
    _check_sort_structure(g, u["tile_bw"] * u["tile_bh"])
    _check_image(g["out_img"])
    o = O.render_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    compare_forward(g, o)
    del g
    gc.collect()
    _compare_gradients(gpu, w, cam, tr, sh, opac, o)


@pytest.mark.parametrize("pose", list(range(8)))
def test_config3_4k_forward_full_size(gpu, pose):
    """6M splats at 3840x2160, forward only (packed RGBA8), each of the eight poses."""
    w_id = 3
    w = CONFIGS[w_id]
    print(f"[case] {w.name} pose {pose}", flush=True)
    tr, sh, opac = _scene(w_id)
    cam = w.camera(pose, 8)
    u = uniforms_for(cam, w.img_w, w.img_h, w.n, w.sh_degree)
    g = gpu_forward(u, tr, sh, opac, 0)
    print(f"[case] {w.name} pose {pose}: visible={g['num_visible']} intersections={g['num_intersections']}",
          flush=True)
    _check_sort_structure(g, u["tile_bw"] * u["tile_bh"])
    _check_subset(g, u, tr, sh, opac, 0, seed=30 + pose, size=10000)
    assert g["out_img"].shape == (w.img_h, w.img_w)


def test_config3_4k_pose_bit_exact(gpu):
    """Config 3's first pose (6M SH3 splats, 3840x2160, forward only): every
    output, the packed RGBA8 image included, bit for bit against the CPU
    restatement."""
    w_id = 3
    w = CONFIGS[w_id]
    print(f"[case] {w.name} pose 0 against the restatement", flush=True)
    tr, sh, opac = _scene(w_id)
    cam = w.camera(0, 8)
    u = uniforms_for(cam, w.img_w, w.img_h, w.n, w.sh_degree)
    g = gpu_forward(u, tr, sh, opac, 0)
    o = O.render_forward(u, tr, sh, opac, 0)
    assert o.num_intersections > 10_000_000
    compare_forward(g, o)
    assert g["out_img"].dtype == np.uint32 and g["out_img"].shape == (w.img_h, w.img_w)
