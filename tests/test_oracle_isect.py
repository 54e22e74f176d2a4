"""Pins the oracle's tile intersection chain against the reference's exact
integer known answers (gsplat_core/test/test.cpp:653-1065), numpy's stable
argsort, and brute-force invariants on random scenes."""
import numpy as np

M2 = np.array([[[20, 20], [50, 50], [8, 8]]], np.float32)
R2 = np.array([[[10, 10], [5, 5], [0, 0]]], np.int32)
D2 = np.array([[1.0, 0.5, 2.0]], np.float32)


def _key(tile, depth_bits):
    return (tile << 32) | depth_bits


def test_known_answers_dense_aabb(oracle):
    # test.cpp:653-737
    out = oracle.isect_tile(M2, R2, D2, 1, 16, 4, 4, sort=True)
    assert out["tiles_per_gauss"].tolist() == [[4, 4, 0]]
    assert ((out["isect_ids"] >> 32) & 0x1F).tolist() == [0, 1, 4, 5, 10, 11, 14, 15]
    assert out["flatten_ids"].tolist() == [0, 0, 0, 0, 1, 1, 1, 1]
    offs = oracle.isect_offset(out["isect_ids"], 1, 4, 4)
    assert offs.shape == (1, 4, 4)
    assert offs.ravel().tolist() == [0, 1, 2, 2, 2, 3, 4, 4, 4, 4, 4, 5, 6, 6, 6, 7]


def test_known_answers_encode(oracle):
    # test.cpp:788-855
    ids, fl = oracle.isect_encode(M2, R2, D2, np.array([[0, 4, 8]], np.int32), 1, 16, 4, 4, 8)
    expect = [_key(t, 0x3F800000) for t in (0, 1, 4, 5)] + [_key(t, 0x3F000000) for t in (10, 11, 14, 15)]
    assert ids.tolist() == expect
    assert fl.tolist() == [0, 0, 0, 0, 1, 1, 1, 1]


def test_known_answers_prefix_sort(oracle):
    # test.cpp:857-1030 (order of Gaussians swapped so the sort reorders)
    m = np.array([[[50, 50], [20, 20], [8, 8]]], np.float32)
    r = np.array([[[5, 5], [10, 10], [0, 0]]], np.int32)
    d = np.array([[0.5, 1.0, 2.0]], np.float32)
    counts = oracle.isect_count(m, r, 16, 4, 4)
    offs, total = oracle.exclusive_scan(counts)
    assert offs.tolist() == [[0, 4, 8]] and total == 8
    ids, fl = oracle.isect_encode(m, r, d, offs, 1, 16, 4, 4, total)
    assert ids.tolist() == [_key(t, 0x3F000000) for t in (10, 11, 14, 15)] + [_key(t, 0x3F800000) for t in (0, 1, 4, 5)]
    sk, sf = oracle.isect_sort(ids, fl)
    assert sk.tolist() == [_key(t, 0x3F800000) for t in (0, 1, 4, 5)] + [_key(t, 0x3F000000) for t in (10, 11, 14, 15)]
    assert sf.tolist() == [1, 1, 1, 1, 0, 0, 0, 0]


def test_known_answer_offsets(oracle):
    # test.cpp:1032-1065
    ids = np.array([_key(t, 0x3F800000) for t in (0, 1, 4, 5)] + [_key(t, 0x3F000000) for t in (10, 11, 14, 15)], np.int64)
    assert oracle.isect_offset(ids, 1, 4, 4).ravel().tolist() == [0, 1, 2, 2, 2, 3, 4, 4, 4, 4, 4, 5, 6, 6, 6, 7]


def test_tile_bits(oracle):
    # gsplat_intersect.cpp:60-65: floor(log2 n) + 1
    for v, b in [(1, 1), (2, 2), (3, 2), (4, 3), (16, 5), (4346, 13), (4096, 13), (8160, 13), (32400, 15)]:
        assert oracle.floor_log2_plus_one(v) == b


def random_projected(rng, I, N, W, H, ties=False):
    means2d = np.stack([rng.uniform(-20, W + 20, (I, N)), rng.uniform(-20, H + 20, (I, N))], -1).astype(np.float32)
    radii = rng.integers(0, 40, size=(I, N, 2)).astype(np.int32)
    radii[rng.random((I, N)) < 0.2] = 0
    depths = rng.uniform(0.1, 20, (I, N)).astype(np.float32)
    if ties:
        depths = np.round(depths).astype(np.float32)  # many equal keys
    return means2d, radii, depths


def test_brute_force_invariants(oracle):
    rng = np.random.default_rng(0)
    I, N, W, H, ts = 3, 500, 150, 100, 16
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    m, r, d = random_projected(rng, I, N, W, H, ties=True)
    out = oracle.isect_tile(m, r, d, I, ts, tw, th, sort=True)
    counts = out["tiles_per_gauss"].ravel()
    keys, fl = out["isect_ids"], out["flatten_ids"]
    assert counts.sum() == keys.size
    assert np.all(np.diff(keys) >= 0)
    assert np.array_equal(np.bincount(fl, minlength=I * N), counts)
    tile_bits = oracle.floor_log2_plus_one(tw * th)
    # every (gaussian, tile) pair of the brute-force AABB test appears exactly once
    mf, rf, df = m.reshape(-1, 2), r.reshape(-1, 2), d.ravel()
    expect = []
    for g in range(I * N):
        if rf[g, 0] <= 0 or rf[g, 1] <= 0:
            continue
        x0 = min(max(0, int(np.floor(np.float32(mf[g, 0] / ts) - np.float32(rf[g, 0] / ts)))), tw)
        x1 = min(max(0, int(np.ceil(np.float32(mf[g, 0] / ts) + np.float32(rf[g, 0] / ts)))), tw)
        y0 = min(max(0, int(np.floor(np.float32(mf[g, 1] / ts) - np.float32(rf[g, 1] / ts)))), th)
        y1 = min(max(0, int(np.ceil(np.float32(mf[g, 1] / ts) + np.float32(rf[g, 1] / ts)))), th)
        bits = int(df[g:g + 1].view(np.uint32)[0])
        img = g // N
        for ty in range(y0, y1):
            for tx in range(x0, x1):
                expect.append(((img << (32 + tile_bits)) | ((ty * tw + tx) << 32) | bits, g))
    ek = np.array([e[0] for e in expect], np.int64)
    ef = np.array([e[1] for e in expect], np.int32)
    order = np.argsort(ek, kind="stable")  # numpy's stable sort, independent of the oracle
    assert np.array_equal(keys, ek[order])
    assert np.array_equal(fl, ef[order])
    # offsets equal numpy's lower bound on key >> 32
    offs = oracle.isect_offset(keys, I, tw, th).ravel()
    want = [(i << tile_bits) | t for i in range(I) for t in range(tw * th)]
    assert np.array_equal(offs, np.searchsorted(keys >> 32, np.array(want, np.int64), side="left"))


def test_empty(oracle):
    m = np.zeros((1, 4, 2), np.float32)
    r = np.zeros((1, 4, 2), np.int32)
    d = np.ones((1, 4), np.float32)
    out = oracle.isect_tile(m, r, d, 1, 16, 2, 2)
    assert out["isect_ids"].size == 0 and out["flatten_ids"].size == 0
    assert oracle.isect_offset(out["isect_ids"], 1, 2, 2).ravel().tolist() == [0, 0, 0, 0]
