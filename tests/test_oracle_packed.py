"""Pins the oracle's packed-layout pieces (upstream gsplat's packed=True path,
which the reference rejects at gsplat_intersect.cpp:115-118 and
gsplat_rasterize.cpp:48-51): packed rows are the dense entries of their
(image, Gaussian) pairs, so every packed result must equal the dense result
of an equivalent dense layout with the flatten ids mapped -- checked here
against the dense oracle, which its own tests pin -- plus hand-computed ids."""
import numpy as np
import pytest

from _helpers import projected_scene

TS = 16


def _dense_from_packed(means, radii, depths, image_ids, I, conics=None, opac=None):
    """Row i goes to dense slot (image_ids[i], i) of [I, nnz] arrays; other
    slots are culled (radius 0). Dense flatten id image * nnz + i maps back to i."""
    nnz = means.shape[0]
    m = np.zeros((I, nnz, 2), np.float32)
    r = np.zeros((I, nnz, 2), np.int32)
    d = np.zeros((I, nnz), np.float32)
    co = np.tile(np.array([1.0, 0.0, 1.0], np.float32), (I, nnz, 1))
    op = np.ones((I, nnz), np.float32)
    rows = np.arange(nnz)
    m[image_ids, rows] = means
    r[image_ids, rows] = radii
    d[image_ids, rows] = depths
    if conics is not None:
        co[image_ids, rows] = conics
        op[image_ids, rows] = opac
    return m, r, d, co, op


def test_packed_isect_known_answer(oracle):
    # rows 0 and 2 in image 1, row 1 in image 0 (tile_bits = 5 for 4x4 tiles)
    m = np.array([[20, 20], [50, 50], [20, 20]], np.float32)
    r = np.array([[10, 10], [5, 5], [10, 10]], np.int32)
    d = np.array([1.0, 0.5, 2.0], np.float32)
    img = np.array([1, 0, 1], np.int32)
    out = oracle.isect_tile_packed(m, r, d, img, 2, TS, 4, 4, sort=True)
    assert out["tiles_per_gauss"].tolist() == [4, 4, 4]
    keys = (out["isect_ids"] >> 32).tolist()
    assert keys == [10, 11, 14, 15] + [32 + t for t in (0, 0, 1, 1, 4, 4, 5, 5)]
    assert out["flatten_ids"].tolist() == [1, 1, 1, 1, 0, 2, 0, 2, 0, 2, 0, 2]


@pytest.mark.parametrize("accutile", [False, True])
@pytest.mark.parametrize("sort", [False, True])
def test_packed_isect_equals_dense(oracle, accutile, sort):
    rng = np.random.default_rng(3)
    I, nnz, W, H = 3, 400, 150, 110
    means, radii, conics, opac, depths = projected_scene(rng, 1, nnz, W, H)
    means, radii, conics, opac, depths = means[0], radii[0], conics[0], opac[0], depths[0]
    img = rng.integers(0, I, nnz).astype(np.int32)
    tw, th = (W + TS - 1) // TS, (H + TS - 1) // TS
    kw = {"conics": conics, "opacities": opac} if accutile else {}
    pk = oracle.isect_tile_packed(means, radii, depths, img, I, TS, tw, th, sort=sort, **kw)
    m, r, d, co, op = _dense_from_packed(means, radii, depths, img, I, conics, opac)
    dkw = {"conics": co, "opacities": op} if accutile else {}
    dn = oracle.isect_tile(m, r, d, I, TS, tw, th, sort=sort, **dkw)
    np.testing.assert_array_equal(pk["tiles_per_gauss"], dn["tiles_per_gauss"][img, np.arange(nnz)])
    if sort:  # both stable in their flatten order, which the mapping preserves
        np.testing.assert_array_equal(pk["isect_ids"], dn["isect_ids"])
        np.testing.assert_array_equal(pk["flatten_ids"], dn["flatten_ids"] % nnz)
    else:  # pair-major in different pair orders: compare as per-row lists
        for i in range(nnz):
            np.testing.assert_array_equal(pk["isect_ids"][pk["flatten_ids"] == i],
                                          dn["isect_ids"][dn["flatten_ids"] == img[i] * nnz + i])


def test_packed_projection_ids(oracle):
    # two cameras, three Gaussians; Gaussian 1 lies behind camera 1 (its view
    # flips z), Gaussian 2 is off-screen for both
    means = np.array([[[0.0, 0.0, 4.0], [0.1, 0.0, 3.0], [50.0, 0.0, 4.0]]], np.float32)
    quats = np.tile(np.array([1, 0, 0, 0], np.float32), (1, 3, 1))
    scales = np.full((1, 3, 3), 0.05, np.float32)
    view = np.tile(np.eye(4, dtype=np.float32), (1, 2, 1, 1))
    view[0, 1, :3, 3] = [0.0, 0.0, -3.5]  # camera 1 sits at z = 3.5
    Ks = np.tile(np.array([[100, 0, 32], [0, 100, 32], [0, 0, 1]], np.float32), (1, 2, 1, 1))
    out = oracle.projection_packed_forward(means, view, Ks, 64, 64, quats=quats, scales=scales)
    assert out["camera_ids"].tolist() == [0, 0, 1]
    assert out["gaussian_ids"].tolist() == [0, 1, 0]
    assert out["batch_ids"].tolist() == [0, 0, 0]
    assert out["indptr"].tolist() == [0, 2, 3]
    dense = oracle.projection_forward(means, view, Ks, 64, 64, quats=quats, scales=scales)
    np.testing.assert_array_equal(out["means2d"][2], dense["means2d"][0, 1, 0])
    assert (out["radii"] > 0).all()
