"""CPU oracle for the splatting operator chain -- TEST INFRASTRUCTURE ONLY.

numpy front end over ``oracle/_build/libgsplat_oracle.so`` (built from
``oracle/gsplat_oracle.cpp`` by ``oracle/Makefile``). The shapes, dtypes and
empty-output conventions follow the reference binding
(gsplat_core/binding/binding.cpp:63-443) and C++ API
(gsplat_core/gsplat_*.cpp); the math is the reference ``eval_cpu`` loops, with
projection culling taken from gsplat_projection.metal:249-326.

Only tests/, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import this module, and only as the reference that
results are compared with.

Every function accepts float32 or float64 arrays; float64 inputs select the
float64 instantiation of the same C++ templates (used by finite-difference
checks).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libgsplat_oracle.so")
_lib = None


def build() -> str:
    """Compile the oracle library with its Makefile; returns the .so path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
    return _lib


def build_native(openmp: bool = False) -> str:
    """A CPU-baseline build (bench.py only, never for comparisons): the same
    source at -O3 -march=native, with its OpenMP loops when `openmp`,
    compiled on the host that runs it into a file named for that host's CPU
    and the source (a build for another CPU's instruction set, or of another
    source, is never loaded). Returns its path."""
    import hashlib
    import platform

    model = platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            model += "".join(l for l in f if l.startswith(("model name", "flags")))
    except OSError:
        pass
    h = hashlib.sha1(model.encode())
    for name in ("gsplat_oracle.cpp", "Makefile"):  # a changed source builds anew
        with open(os.path.join(_HERE, name), "rb") as f:
            h.update(f.read())
    tag = h.hexdigest()[:12]
    path = os.path.join(_HERE, "_build", f"libgsplat_oracle_native{'_omp' if openmp else ''}_{tag}.so")
    if not os.path.exists(path):
        subprocess.run(["make", "-s", "-C", _HERE, "native", f"NATIVE={path}"] + (["OMP=1"] if openmp else []),
                       check=True)
    return path


def flush_denormals() -> bool:
    """CPU baseline only: flush denormals to zero on this thread and the
    OpenMP threads (as a tuned CPU run would); True where supported."""
    f = lib().oracle_flush_denormals
    f.restype = ctypes.c_int
    return bool(f())


def use_library(path: str) -> None:
    """Routes every function of this module to the library at `path`."""
    global _lib
    _lib = ctypes.CDLL(path)


def set_threads(n: int) -> int:
    """Threads of the OpenMP loops (n <= 0 keeps the current count); returns
    the count in effect (1 for the tests' single-threaded build)."""
    f = lib().oracle_set_threads
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_int]
    return int(f(int(n)))


def _sfx(dtype) -> str:
    return "f64" if np.dtype(dtype) == np.float64 else "f32"


def _ptr(a):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    if a is None:
        return None
    return np.ascontiguousarray(a, dtype=dtype)


def _fn(name):
    f = getattr(lib(), name)
    f.restype = None
    return f


class ProjParams(ctypes.Structure):
    _fields_ = [
        ("image_width", ctypes.c_int32),
        ("image_height", ctypes.c_int32),
        ("eps2d", ctypes.c_float),
        ("near_plane", ctypes.c_float),
        ("far_plane", ctypes.c_float),
        ("radius_clip", ctypes.c_float),
        ("calc_compensations", ctypes.c_int32),
        ("camera_model", ctypes.c_int32),
        ("use_covars", ctypes.c_int32),
        ("use_opacities", ctypes.c_int32),
    ]


I64 = ctypes.c_int64


# ---------------------------------------------------------------- quat/scale
def quat_scale_to_covar_preci_forward(quats, scales, compute_covar=True, compute_preci=True, triu=True):
    """gsplat_quat_scale_to_covar.cpp:337-354 (shapes), :374-405 (math)."""
    dt = np.asarray(quats).dtype
    q = _c(quats, dt)
    s = _c(scales, dt)
    n = q.size // 4
    tail = (6,) if triu else (3, 3)
    shape = q.shape[:-1] + tail
    covars = np.zeros(shape if compute_covar else (0,), dt)
    precis = np.zeros(shape if compute_preci else (0,), dt)
    _fn(f"oracle_quat_scale_to_covar_preci_fwd_{_sfx(dt)}")(
        _ptr(q), _ptr(s), I64(n), int(compute_covar), int(compute_preci), int(triu), _ptr(covars), _ptr(precis))
    return covars, precis


def quat_scale_to_covar_preci_backward(quats, scales, v_covars=None, v_precis=None, triu=True):
    """gsplat_quat_scale_to_covar.cpp:356-372, :407-468."""
    dt = np.asarray(quats).dtype
    q = _c(quats, dt)
    s = _c(scales, dt)
    vc = _c(v_covars, dt) if v_covars is not None and np.size(v_covars) else None
    vp = _c(v_precis, dt) if v_precis is not None and np.size(v_precis) else None
    n = q.size // 4
    v_quats = np.zeros(q.shape, dt)
    v_scales = np.zeros(s.shape, dt)
    _fn(f"oracle_quat_scale_to_covar_preci_bwd_{_sfx(dt)}")(
        _ptr(q), _ptr(s), _ptr(vc), _ptr(vp), I64(n), int(triu), _ptr(v_quats), _ptr(v_scales))
    return v_quats, v_scales


# ---------------------------------------------------------------- projection
def _proj_dims(means, viewmats):
    N = means.shape[-2]
    C = viewmats.shape[-3]
    B = means.size // (N * 3) if N else int(np.prod(means.shape[:-2]))
    return B, C, N


def projection_forward(means, viewmats, Ks, image_width, image_height, covars=None, quats=None,
                       scales=None, opacities=None, eps2d=0.3, near_plane=0.01, far_plane=1e10,
                       radius_clip=0.0, calc_compensations=False, camera_model=0):
    """Forward projection; outputs as gsplat_projection.cpp:584-618."""
    dt = np.asarray(means).dtype
    m = _c(means, dt)
    vm = _c(viewmats, dt)
    K = _c(Ks, dt)
    use_covars = covars is not None and np.size(covars) > 0
    use_opac = opacities is not None and np.size(opacities) > 0
    cv = _c(covars, dt) if use_covars else None
    q = None if use_covars else _c(quats, dt)
    s = None if use_covars else _c(scales, dt)
    op = _c(opacities, dt) if use_opac else None
    B, C, N = _proj_dims(m, vm)
    prefix = m.shape[:-2] + (C, N)
    radii = np.zeros(prefix + (2,), np.int32)
    means2d = np.zeros(prefix + (2,), dt)
    depths = np.zeros(prefix, dt)
    conics = np.zeros(prefix + (3,), dt)
    comps = np.zeros(prefix if calc_compensations else (0,), dt)
    p = ProjParams(image_width, image_height, eps2d, near_plane, far_plane, radius_clip,
                   int(calc_compensations), camera_model, int(use_covars), int(use_opac))
    _fn(f"oracle_projection_fwd_{_sfx(dt)}")(
        _ptr(m), _ptr(cv), _ptr(q), _ptr(s), _ptr(op), _ptr(vm), _ptr(K), I64(B), I64(C), I64(N),
        ctypes.byref(p), _ptr(radii), _ptr(means2d), _ptr(depths), _ptr(conics),
        _ptr(comps) if calc_compensations else None)
    return {"radii": radii, "means2d": means2d, "depths": depths, "conics": conics, "compensations": comps}


def projection_backward(means, viewmats, Ks, image_width, image_height, radii, conics, v_means2d,
                        v_depths, v_conics, covars=None, quats=None, scales=None, compensations=None,
                        v_compensations=None, eps2d=0.3, camera_model=0, viewmats_requires_grad=False):
    """gsplat_projection.cpp:620-652 (shapes), :965-1121 (math)."""
    dt = np.asarray(means).dtype
    m = _c(means, dt)
    vm = _c(viewmats, dt)
    K = _c(Ks, dt)
    use_covars = covars is not None and np.size(covars) > 0
    cv = _c(covars, dt) if use_covars else None
    q = None if use_covars else _c(quats, dt)
    s = None if use_covars else _c(scales, dt)
    calc = compensations is not None and np.size(compensations) > 0
    vcomp = v_compensations is not None and np.size(v_compensations) > 0
    B, C, N = _proj_dims(m, vm)
    v_means = np.zeros(m.shape, dt)
    v_covars = np.zeros(cv.shape if use_covars else (0,), dt)
    v_quats = np.zeros((0,) if use_covars else q.shape, dt)
    v_scales = np.zeros((0,) if use_covars else s.shape, dt)
    v_viewmats = np.zeros(vm.shape if viewmats_requires_grad else (0,), dt)
    p = ProjParams(image_width, image_height, eps2d, -1e20, 1e20, 0.0, int(calc), camera_model,
                   int(use_covars), 0)
    _fn(f"oracle_projection_bwd_{_sfx(dt)}")(
        _ptr(m), _ptr(cv), _ptr(q), _ptr(s), _ptr(vm), _ptr(K), I64(B), I64(C), I64(N), ctypes.byref(p),
        _ptr(_c(radii, np.int32)), _ptr(_c(conics, dt)), _ptr(_c(compensations, dt)) if calc else None,
        _ptr(_c(v_means2d, dt)), _ptr(_c(v_depths, dt)), _ptr(_c(v_conics, dt)),
        _ptr(_c(v_compensations, dt)) if vcomp else None,
        _ptr(v_means), _ptr(v_covars) if use_covars else None, None if use_covars else _ptr(v_quats),
        None if use_covars else _ptr(v_scales), _ptr(v_viewmats) if viewmats_requires_grad else None)
    out = {"v_means": v_means}
    if use_covars:
        out["v_covars"] = v_covars
    else:
        out["v_quats"] = v_quats
        out["v_scales"] = v_scales
    if viewmats_requires_grad:
        out["v_viewmats"] = v_viewmats
    return out


# ---------------------------------------------------------------------- SH
def sh_forward(degree, dirs, coeffs, masks=None):
    """gsplat_spherical_harmonics.cpp:429-441, :466-501."""
    dt = np.asarray(dirs).dtype
    d = _c(dirs, dt)
    co = _c(coeffs, dt)
    K = co.shape[-2]
    n = d.size // 3
    mk = np.ascontiguousarray(masks, dtype=np.uint8) if masks is not None and np.size(masks) else None
    colors = np.zeros(d.shape, dt)
    _fn(f"oracle_sh_fwd_{_sfx(dt)}")(int(degree), _ptr(d), _ptr(co), _ptr(mk), I64(n), I64(K), _ptr(colors))
    return colors


def sh_backward(degree, dirs, coeffs, v_colors, masks=None, compute_v_dirs=True):
    """gsplat_spherical_harmonics.cpp:443-464, :503-554."""
    dt = np.asarray(dirs).dtype
    d = _c(dirs, dt)
    co = _c(coeffs, dt)
    K = co.shape[-2]
    n = d.size // 3
    mk = np.ascontiguousarray(masks, dtype=np.uint8) if masks is not None and np.size(masks) else None
    v_dirs = np.zeros(d.shape if compute_v_dirs else (0,), dt)
    v_coeffs = np.zeros(co.shape, dt)
    _fn(f"oracle_sh_bwd_{_sfx(dt)}")(int(degree), _ptr(d), _ptr(co), _ptr(mk), _ptr(_c(v_colors, dt)), I64(n),
                                     I64(K), _ptr(v_dirs) if compute_v_dirs else None, _ptr(v_coeffs))
    return v_dirs, v_coeffs


# ----------------------------------------------------------------- isect
def floor_log2_plus_one(value: int) -> int:
    f = lib().oracle_floor_log2_plus_one
    f.restype = ctypes.c_int
    return f(int(value))


def isect_count(means2d, radii, tile_size, tile_width, tile_height):
    m = _c(means2d, np.float32)
    r = _c(radii, np.int32)
    out = np.zeros(m.shape[:-1], np.int32)
    _fn("oracle_isect_count")(_ptr(m), _ptr(r), I64(out.size), tile_size, tile_width, tile_height, _ptr(out))
    return out


def exclusive_scan(counts):
    c = _c(counts, np.int32)
    out = np.zeros(c.shape, np.int32)
    f = lib().oracle_exclusive_scan
    f.restype = ctypes.c_int64
    total = f(_ptr(c), I64(c.size), _ptr(out))
    return out, int(total)


def isect_encode(means2d, radii, depths, offsets, I, tile_size, tile_width, tile_height, total):
    m = _c(means2d, np.float32)
    r = _c(radii, np.int32)
    d = _c(depths, np.float32)
    o = _c(offsets, np.int32)
    ids = np.zeros(total, np.int64)
    fl = np.zeros(total, np.int32)
    f = lib().oracle_isect_encode
    f.restype = ctypes.c_int
    rc = f(_ptr(m), _ptr(r), _ptr(d), _ptr(o), I64(I), I64(d.size), tile_size, tile_width, tile_height,
           I64(total), _ptr(ids), _ptr(fl))
    if rc != 0:
        raise RuntimeError("intersect_tile_encode tile_offsets write out of bounds.")
    return ids, fl


def isect_count_accutile(means2d, radii, conics, opacities, tile_size, tile_width, tile_height):
    """Ellipse (AccuTile) tile counts; the restated method is described in gsplat_oracle.cpp."""
    m = _c(means2d, np.float32)
    r = _c(radii, np.int32)
    co = _c(conics, np.float32)
    op = _c(opacities, np.float32)
    out = np.zeros(m.shape[:-1], np.int32)
    _fn("oracle_isect_count_accutile")(_ptr(m), _ptr(r), _ptr(co), _ptr(op), I64(out.size), tile_size, tile_width,
                                       tile_height, _ptr(out))
    return out


def isect_encode_accutile(means2d, radii, conics, opacities, depths, offsets, I, tile_size, tile_width,
                          tile_height, total):
    m = _c(means2d, np.float32)
    r = _c(radii, np.int32)
    co = _c(conics, np.float32)
    op = _c(opacities, np.float32)
    d = _c(depths, np.float32)
    o = _c(offsets, np.int32)
    ids = np.zeros(total, np.int64)
    fl = np.zeros(total, np.int32)
    f = lib().oracle_isect_encode_accutile
    f.restype = ctypes.c_int
    rc = f(_ptr(m), _ptr(r), _ptr(co), _ptr(op), _ptr(d), _ptr(o), I64(I), I64(d.size), tile_size, tile_width,
           tile_height, I64(total), _ptr(ids), _ptr(fl))
    if rc != 0:
        raise RuntimeError("intersect_tile_encode tile_offsets write out of bounds.")
    return ids, fl


def isect_sort(isect_ids, flatten_ids):
    k = _c(isect_ids, np.int64)
    v = _c(flatten_ids, np.int32)
    ko = np.zeros_like(k)
    vo = np.zeros_like(v)
    _fn("oracle_isect_sort")(_ptr(k), _ptr(v), I64(k.size), _ptr(ko), _ptr(vo))
    return ko, vo


def isect_tile(means2d, radii, depths, I, tile_size, tile_width, tile_height, sort=True, conics=None,
               opacities=None):
    """gsplat_intersect.cpp:288-307: count -> scan -> total -> encode -> sort; with conics and
    opacities the ellipse (AccuTile) tiles."""
    if conics is not None:
        counts = isect_count_accutile(means2d, radii, conics, opacities, tile_size, tile_width, tile_height)
        offsets, total = exclusive_scan(counts)
        ids, fl = isect_encode_accutile(means2d, radii, conics, opacities, depths, offsets, I, tile_size,
                                        tile_width, tile_height, total)
    else:
        counts = isect_count(means2d, radii, tile_size, tile_width, tile_height)
        offsets, total = exclusive_scan(counts)
        ids, fl = isect_encode(means2d, radii, depths, offsets, I, tile_size, tile_width, tile_height, total)
    if sort:
        ids, fl = isect_sort(ids, fl)
    return {"tiles_per_gauss": counts, "isect_ids": ids, "flatten_ids": fl}


def isect_tile_packed(means2d, radii, depths, image_ids, I, tile_size, tile_width, tile_height, sort=True,
                      conics=None, opacities=None):
    """Packed layout: nnz rows, row i in image image_ids[i], flatten ids = rows; AABB or
    (conics + opacities) ellipse tiles; count -> scan -> encode -> stable sort."""
    m = _c(means2d, np.float32)
    r = _c(radii, np.int32)
    d = _c(depths, np.float32)
    img = _c(image_ids, np.int32)
    if conics is not None:
        counts = isect_count_accutile(m, r, conics, opacities, tile_size, tile_width, tile_height)
        co, op = _c(conics, np.float32), _c(opacities, np.float32)
    else:
        counts = isect_count(m, r, tile_size, tile_width, tile_height)
        co = op = None
    offsets, total = exclusive_scan(counts)
    ids = np.zeros(total, np.int64)
    fl = np.zeros(total, np.int32)
    f = lib().oracle_isect_encode_packed
    f.restype = ctypes.c_int
    rc = f(_ptr(m), _ptr(r), _ptr(co), _ptr(op), _ptr(img), _ptr(d), _ptr(_c(offsets, np.int32)), I64(d.size),
           tile_size, tile_width, tile_height, I64(total), _ptr(ids), _ptr(fl))
    if rc != 0:
        raise RuntimeError("intersect_tile_encode tile_offsets write out of bounds.")
    if sort:
        ids, fl = isect_sort(ids, fl)
    return {"tiles_per_gauss": counts, "isect_ids": ids, "flatten_ids": fl}


def projection_packed_forward(means, viewmats, Ks, W, H, **kw):
    """Packed layout of the projection (upstream's fully_fused_projection(packed=True)):
    the dense oracle's outputs at the visible pairs (both radii > 0), ordered by
    (batch, camera, gaussian), with their ids and each camera's first row."""
    e = projection_forward(means, viewmats, Ks, W, H, **kw)
    radii = e["radii"]
    vis = np.all(radii > 0, axis=-1)  # [..., C, N]
    C, N = vis.shape[-2], vis.shape[-1]
    flat = np.flatnonzero(vis.reshape(-1))
    cam, n = flat // N, flat % N
    counts = np.bincount(cam, minlength=vis.size // N)
    out = {"batch_ids": (cam // C).astype(np.int32), "camera_ids": (cam % C).astype(np.int32),
           "gaussian_ids": n.astype(np.int32),
           "indptr": np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)}
    for k in ("radii", "means2d", "depths", "conics", "compensations"):
        if k in e and e[k] is not None and np.size(e[k]):
            v = e[k]
            out[k] = v.reshape((vis.size,) + v.shape[vis.ndim:])[flat]
    return out


def isect_offset(isect_ids, I, tile_width, tile_height):
    """gsplat_intersect.cpp:586-641."""
    k = _c(isect_ids, np.int64)
    out = np.zeros((I, tile_height, tile_width), np.int32)
    _fn("oracle_isect_offset")(_ptr(k), I64(k.size), I, tile_width, tile_height, _ptr(out))
    return out


# ------------------------------------------------------------- rasterize
def raster_indices(means2d, conics, opacities, tile_offsets, flatten_ids, image_width, image_height, tile_size,
                   range_start=0, range_end=2**40, transmittances=None):
    """rasterize_to_indices: (gaussian_ids int32 [M], indices int64 [M]), pixel-major."""
    to = _c(tile_offsets, np.int32)
    th, tw = to.shape[-2], to.shape[-1]
    I = to.size // (th * tw)
    m, co, op = _c(means2d, np.float32), _c(conics, np.float32), _c(opacities, np.float32)
    fl = _c(flatten_ids, np.int32)
    tr = _c(transmittances, np.float32) if transmittances is not None else None
    n_pix = I * image_width * image_height
    counts = np.zeros(n_pix, np.int32)
    f = lib().oracle_raster_indices
    args = (I64(range_start), I64(range_end), _ptr(tr), _ptr(m), _ptr(co), _ptr(op), _ptr(to), _ptr(fl), I64(I),
            image_width, image_height, tile_size, tw, th, I64(fl.size))
    f(*args, _ptr(counts), None, None, None)
    starts, total = exclusive_scan(counts)
    gids = np.zeros(total, np.int32)
    idx = np.zeros(total, np.int64)
    f(*args, None, _ptr(starts), _ptr(gids), _ptr(idx))
    return gids, idx


def _raster_dims(means2d, colors, tile_offsets):
    th, tw = tile_offsets.shape[-2], tile_offsets.shape[-1]
    I = tile_offsets.size // (th * tw)
    N = means2d.shape[-2]
    ch = colors.shape[-1]
    return I, N, ch, tw, th


def raster_forward(means2d, conics, colors, opacities, tile_offsets, flatten_ids, image_width, image_height,
                   tile_size, backgrounds=None, masks=None):
    """gsplat_rasterize.cpp:165-208 (shapes), :249-369 (math)."""
    dt = np.asarray(means2d).dtype
    to = _c(tile_offsets, np.int32)
    I, N, ch, tw, th = _raster_dims(np.asarray(means2d), np.asarray(colors), to)
    prefix = to.shape[:-2]
    rc = np.zeros(prefix + (image_height, image_width, ch), dt)
    ra = np.zeros(prefix + (image_height, image_width, 1), dt)
    li = np.zeros(prefix + (image_height, image_width), np.int32)
    bg = _c(backgrounds, dt) if backgrounds is not None and np.size(backgrounds) else None
    mk = np.ascontiguousarray(masks, dtype=np.uint8) if masks is not None and np.size(masks) else None
    fl = _c(flatten_ids, np.int32)
    ev = np.zeros(to.shape, np.int64)
    _fn(f"oracle_raster_fwd_{_sfx(dt)}")(
        _ptr(_c(means2d, dt)), _ptr(_c(conics, dt)), _ptr(_c(colors, dt)), _ptr(_c(opacities, dt)), _ptr(bg),
        _ptr(mk), _ptr(to), _ptr(fl), I64(I), I64(ch), image_width, image_height, tile_size, tw, th,
        I64(fl.size), _ptr(rc), _ptr(ra), _ptr(li), _ptr(ev))
    # tile_evals: per tile, the forward loop's iterations over its pixels
    # (entries evaluated up to each pixel's termination, E_f)
    return {"render_colors": rc, "render_alphas": ra, "last_ids": li, "tile_evals": ev}


def raster_backward(means2d, conics, colors, opacities, tile_offsets, flatten_ids, image_width, image_height,
                    tile_size, render_alphas, last_ids, v_render_colors, v_render_alphas, backgrounds=None,
                    masks=None, absgrad=False):
    """gsplat_rasterize.cpp:210-247 (shapes), :371-569 (math)."""
    dt = np.asarray(means2d).dtype
    to = _c(tile_offsets, np.int32)
    m2 = _c(means2d, dt)
    co = _c(colors, dt)
    I, N, ch, tw, th = _raster_dims(m2, co, to)
    bg = _c(backgrounds, dt) if backgrounds is not None and np.size(backgrounds) else None
    mk = np.ascontiguousarray(masks, dtype=np.uint8) if masks is not None and np.size(masks) else None
    fl = _c(flatten_ids, np.int32)
    v_abs = np.zeros(m2.shape if absgrad else (0,), dt)
    v_m = np.zeros(m2.shape, dt)
    v_c = np.zeros(np.shape(conics), dt)
    v_col = np.zeros(co.shape, dt)
    v_op = np.zeros(np.shape(opacities), dt)
    v_bg = np.zeros(bg.shape if bg is not None else (0,), dt)
    _fn(f"oracle_raster_bwd_{_sfx(dt)}")(
        _ptr(m2), _ptr(_c(conics, dt)), _ptr(co), _ptr(_c(opacities, dt)), _ptr(bg), _ptr(mk), _ptr(to), _ptr(fl),
        I64(I), I64(N), I64(ch), image_width, image_height, tile_size, tw, th, I64(fl.size),
        _ptr(_c(render_alphas, dt)), _ptr(_c(last_ids, np.int32)), _ptr(_c(v_render_colors, dt)),
        _ptr(_c(v_render_alphas, dt)), _ptr(v_abs) if absgrad else None, _ptr(v_m), _ptr(v_c), _ptr(v_col),
        _ptr(v_op), _ptr(v_bg) if bg is not None else None)
    out = {"v_means2d": v_m, "v_conics": v_c, "v_colors": v_col, "v_opacities": v_op}
    if absgrad:
        out["v_means2d_abs"] = v_abs
    if bg is not None:
        out["v_backgrounds"] = v_bg
    return out

