"""CPU oracle of the training step's image loss -- TEST INFRASTRUCTURE ONLY.

numpy float64 restatement of scanner_points_training_utils.py:1123-1172:
  local_average(image, ws)        :1123-1128  conv2d of each channel with a
                                  ws x ws box of ones / ws^2, zero padding
                                  ws // 2 (NHWC, map [B, Ho, Wo, C] with
                                  Ho = H + 2 (ws // 2) - ws + 1); the weight
                                  ones / ws^2 is built in the image's dtype
                                  (:1125-1126), so float32 images carry the
                                  float32 rounding of 1 / ws^2 (a common
                                  factor of every box mean, which moves the
                                  SSIM mean by about 1e-5 relative)
  ssim_index(image, target, ws)   :1131-1144
  image_loss_components(...)      :1147-1172  (L1, ssim, dssim = (1 - ssim) / 2,
                                  loss = (1 - lambda) L1 + lambda dssim)
and the VJP of the L1 and SSIM terms with respect to the image
(`image_loss_vjp`), written out from the chain rule:
  with N1 = 2 mu_x mu_y + c1, N2 = 2 s_xy + c2, D1 = mu_x^2 + mu_y^2 + c1,
  D2 = s_xx + s_yy + c2, S = N1 N2 / max(D1 D2, 1e-12):
  dS/dmu_x = 2 mu_y (N2 - N1) / D + 2 mu_x (-S / D1 + S / D2),
  dS/dE[x^2] = -S / D2, dS/dE[xy] = 2 N1 / D  (D = D1 D2; the D1, D2 terms
  vanish where the max picks 1e-12),
  d mean(S) / dx[p] = (1 / (n_map ws^2)) sum over the map positions q whose
  window holds p of (dS/dmu_x + 2 x[p] dS/dE[x^2] + y[p] dS/dE[xy]) (q).
The float64 arithmetic here stands in for the reference's float32 MLX
kernels; the checks in tests/test_oracle_image_loss.py pin it: the box means
against scipy.ndimage.uniform_filter and torch's avg_pool2d, the SSIM map
against a per-window brute-force loop, closed forms (identical images give
S = 1; constant images give (2ab + c1) / (a^2 + b^2 + c1) inside), the
reference's own image_loss_debug.py assertions, and the VJP against central
finite differences.

Only tests/, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import this module, and only as the reference that
results are compared with.
"""
from __future__ import annotations

import numpy as np

C1 = 0.01 * 0.01
C2 = 0.03 * 0.03
MIN_DEN = 1.0e-12


def _window_sum(a: np.ndarray, ws: int, lo: int, hi: int) -> np.ndarray:
    """Sum of a [B, H, W, C] array over ws x ws windows after padding rows and
    columns with `lo` zeros before and `hi` after (separable: rows, then
    columns)."""
    p = np.pad(np.asarray(a, np.float64), ((0, 0), (lo, hi), (lo, hi), (0, 0)))
    rows = np.lib.stride_tricks.sliding_window_view(p, ws, axis=1).sum(-1)
    return np.lib.stride_tricks.sliding_window_view(rows, ws, axis=2).sum(-1)


def box_weight(image, ws: int) -> float:
    """ones / ws^2 in the image's dtype (float32 unless given float64)."""
    dt = np.float64 if np.asarray(image).dtype == np.float64 else np.float32
    return float(dt(1.0) / dt(ws * ws))


def local_average(image, ws: int) -> np.ndarray:
    """:1123-1128 -- box mean, zero padding ws // 2."""
    pad = ws // 2
    return _window_sum(image, ws, pad, pad) * box_weight(image, ws)


def _stats(image, target, ws):
    w, pad = box_weight(image, ws), ws // 2
    x = np.asarray(image, np.float64)
    y = np.asarray(target, np.float64)

    def avg(a):
        return _window_sum(a, ws, pad, pad) * w

    mu_x = avg(x)
    mu_y = avg(y)
    mu_x2, mu_y2, mu_xy = mu_x * mu_x, mu_y * mu_y, mu_x * mu_y
    s_xx = avg(x * x) - mu_x2
    s_yy = avg(y * y) - mu_y2
    s_xy = avg(x * y) - mu_xy
    n1 = 2.0 * mu_xy + C1
    n2 = 2.0 * s_xy + C2
    d1 = mu_x2 + mu_y2 + C1
    d2 = s_xx + s_yy + C2
    return mu_x, mu_y, n1, n2, d1, d2


def ssim_map(image, target, ws: int) -> np.ndarray:
    """The SSIM map of :1131-1144 before the mean, [B, Ho, Wo, C]."""
    _, _, n1, n2, d1, d2 = _stats(image, target, ws)
    return (n1 * n2) / np.maximum(d1 * d2, MIN_DEN)


def ssim_index(image, target, ws: int) -> float:
    """:1131-1144."""
    return float(np.mean(ssim_map(image, target, ws)))


def l1(image, target) -> float:
    return float(np.mean(np.abs(np.asarray(image, np.float64) - np.asarray(target, np.float64))))


def image_loss_components(image, target, loss_mode: str, ssim_lambda: float, ssim_window_size: int) -> dict:
    """:1147-1172."""
    v_l1 = l1(image, target)
    if loss_mode == "l1":
        return {"loss": v_l1, "l1": v_l1, "ssim": 1.0, "dssim": 0.0}
    if loss_mode != "l1_dssim":
        raise ValueError(f"Unsupported loss mode: {loss_mode}")
    ssim = ssim_index(image, target, ssim_window_size)
    dssim = (1.0 - ssim) * 0.5
    return {"loss": (1.0 - ssim_lambda) * v_l1 + ssim_lambda * dssim, "l1": v_l1, "ssim": ssim, "dssim": dssim}


def ssim_vjp(image, target, ws: int, g_ssim: float = 1.0) -> np.ndarray:
    """g_ssim * d ssim_index / d image, [B, H, W, C] float64."""
    t_mu, t_xx, t_xy, scale = ssim_vjp_terms(image, target, ws)
    return g_ssim * (t_mu + t_xx + t_xy) * scale


def ssim_vjp_terms(image, target, ws: int, transposed: bool = True):
    """The three terms of d ssim_index / d image before the common factor
    1 / (n_map ws^2): through mu_x, through E[x^2] and through E[xy]; and that
    factor (with the box weight of the image's dtype). transposed=False gathers with the forward's window instead of its
    transpose (the same for odd ws; kept for tests that show the difference)."""
    x = np.asarray(image, np.float64)
    y = np.asarray(target, np.float64)
    mu_x, mu_y, n1, n2, d1, d2 = _stats(x, y, ws)
    den = d1 * d2
    used = den > MIN_DEN
    dd = np.where(used, den, MIN_DEN)
    s = n1 * n2 / dd
    dn1, dn2 = n2 / dd, n1 / dd
    dd1 = np.where(used, -s / d1, 0.0)
    dd2 = np.where(used, -s / d2, 0.0)
    a = 2.0 * mu_y * (dn1 - dn2) + 2.0 * mu_x * (dd1 - dd2)
    b = dd2
    c = 2.0 * dn2
    # transposed window: input p collects the map positions q in
    # [p + pad - ws + 1, p + pad], i.e. the first H x W window sums after
    # padding the map with ws - 1 - pad zeros before and pad after (the map
    # has one more row and column than the image for even ws)
    pad = ws // 2
    lo, hi = (ws - 1 - pad, pad) if transposed else (pad, ws - 1 - pad)
    H, W = x.shape[1], x.shape[2]
    sa, sb, sc = (_window_sum(t, ws, lo, hi)[:, :H, :W] for t in (a, b, c))
    return sa, 2.0 * x * sb, y * sc, box_weight(image, ws) / a.size


def l1_vjp(image, target, g_l1: float = 1.0) -> np.ndarray:
    x = np.asarray(image, np.float64)
    y = np.asarray(target, np.float64)
    return g_l1 * np.sign(x - y) / x.size


def image_loss_vjp(image, target, ws: int, g_l1: float = 0.0, g_ssim: float = 0.0) -> np.ndarray:
    """The image cotangent of the (L1, ssim) pair for cotangents (g_l1, g_ssim)."""
    return l1_vjp(image, target, g_l1) + ssim_vjp(image, target, ws, g_ssim)


def loss_vjp(image, target, loss_mode: str, ssim_lambda: float, ssim_window_size: int, g: float = 1.0):
    """The image cotangent of image_loss_components(...)["loss"]."""
    if loss_mode == "l1":
        return l1_vjp(image, target, g)
    return image_loss_vjp(image, target, ssim_window_size, g_l1=g * (1.0 - ssim_lambda),
                          g_ssim=-0.5 * ssim_lambda * g)
