"""Closed-form known answers for three reference behaviours that seeded random
scenes never reach.  The expected values are computed here, from numbers.
Neither the oracle nor the HIP kernels are imported.  ``test_oracle_pins.py``
checks the oracle against them (CPU) and ``test_gpu_known_answers.py`` checks
the HIP kernels (GPU).

* The alpha ceiling: alpha = min(sigmoid(o) * exp(-D / 2), 0.99)
  (reference src/gaussian_splats/kernels/rasterize/torch.py:205,
  composite.py:81).  The gradient through the ceiling is zero
  (composite_bwd.py:149).
* Colour has a lower clamp only: rgb = max(sum_k B_k c_k + 0.5, 0)
  (splats/utils.py:75).  A colour above 1 stays above 1.
* The EWA Jacobian clamps x/d and y/d at +-1.3 * tan(half field of view)
  (splats/camera.py:106-119).  No gradient passes through a clamped ratio.

Scene "peak": one Gaussian at an integer pixel, opacity logit 6.  Its
alpha0 = sigmoid(6) = 0.99753 exceeds the ceiling at the centre pixel.  Its
DC colour is (1.7, 1.0, -0.3 -> 0).  The camera is the identity with
fx = fy = 40 and a 32 x 24 image, principal point (16, 12).  The Gaussian
sits at mean (0, 0, -2), depth d = 2.  Its screen variance is
(fx/d * s)^2 + 0.03 = (20 * 0.1)^2 + 0.03 = 4.03, isotropic.

Scene "jacobian": six isotropic Gaussians (s = 0.1, identity rotation) at
depth 2 in front of an identity camera.  fx = fy = 100 and the image is
100 x 80, so the clamps are lx = 1.3 * 100 / 200 = 0.65 and
ly = 1.3 * 80 / 200 = 0.52.  With J = [[50, 0, 50 xc], [0, -50, -50 yc]],
xc = clamp(x/d, +-lx) and yc = clamp(y/d, +-ly), the 2-D covariance is
Sigma = 0.01 J J^T + 0.03 I:
  Sigma00 = 25 (1 + xc^2) + 0.03
  Sigma01 = -25 xc yc
  Sigma11 = 25 (1 + yc^2) + 0.03
"""

from __future__ import annotations

import math

import numpy as np

SH_C0 = 0.28209479177387814  # 1 / (2 sqrt(pi)), the degree-0 real SH constant


def sigmoid(x: float) -> float:
    return 1.0 / (1.0 + math.exp(-x))


# ---------------------------------------------------------------- "peak" scene
PEAK = dict(
    fx=40.0, fy=40.0, cx=16.0, cy=12.0, width=32, height=24,
    mean=(0.0, 0.0, -2.0), rotation=(1.0, 0.0, 0.0, 0.0), log_scale=math.log(0.1),
    opacity_logit=6.0,
    # DC coefficients: SH_C0 * c + 0.5 = (1.7, 1.0, -0.3).
    dc=(1.2 / SH_C0, 0.5 / SH_C0, -0.8 / SH_C0),
    centre=(16, 12),  # (x, y) pixel at the projected mean
)
PEAK_RGB = np.array([1.7, 1.0, 0.0])
PEAK_VAR = (40.0 / 2.0 * 0.1) ** 2 + 0.03  # 4.03
PEAK_ALPHA0 = sigmoid(6.0)


def peak_alpha() -> np.ndarray:
    """[H, W] blended alpha of the peak scene: min(alpha0 e^{-D/2}, 0.99), 0 below 1/255."""
    ys, xs = np.mgrid[0:PEAK["height"], 0:PEAK["width"]]
    d2 = ((xs - 16.0) ** 2 + (ys - 12.0) ** 2) / PEAK_VAR
    a = np.minimum(PEAK_ALPHA0 * np.exp(-0.5 * d2), 0.99)
    return np.where(a >= 1.0 / 255.0, a, 0.0)


def peak_image() -> np.ndarray:
    return peak_alpha()[..., None] * PEAK_RGB


def peak_transmittance() -> np.ndarray:
    return 1.0 - peak_alpha()


# Gradients of L = sum_c image[12, 16, c] (the clamped centre pixel): alpha is
# the constant 0.99 there, so only the colour receives a gradient, and only in
# the two unclamped channels.
PEAK_CENTRE_GRAD_DC = 0.99 * SH_C0 * np.array([1.0, 1.0, 0.0])

# Gradients of L = sum_c image[12, 17, c], one pixel right of the centre:
# alpha = alpha0 e^{-1/(2 var)} < 0.99 is not clamped.
PEAK_RIGHT_ALPHA = PEAK_ALPHA0 * math.exp(-0.5 / PEAK_VAR)
PEAK_RIGHT_GRAD_LOGIT = PEAK_ALPHA0 * (1 - PEAK_ALPHA0) * math.exp(-0.5 / PEAK_VAR) * 2.7
# dalpha/du = alpha (x - u) / var with x - u = 1; du/dmean_x = fx / d = 20.
# Sigma does not depend on mean_x at x/d = 0 (d Sigma00 / d px = 2 s^2 fx^2 px / d^4 = 0).
# The pixel has dy = 0, so D = 1 / Sigma00 with Sigma00 = s0^2 (fx/d)^2 + 0.03:
#   dL/dSigma00 = 2.7 alpha / (2 var^2);
#   dSigma00/dmean_z = -dSigma00/dd = 2 s0^2 fx^2 / d^3 = 4;
#   dSigma00/dlog s0 = 2 s0^2 fx^2 / d^2 = 8.
# Nothing depends on mean_y (v = y there), log s1, log s2 or the rotation.
PEAK_RIGHT_GRAD_MEAN = np.array([
    20.0 * PEAK_RIGHT_ALPHA / PEAK_VAR * 2.7,
    0.0,
    2.7 * PEAK_RIGHT_ALPHA / (2 * PEAK_VAR**2) * 4.0,
])
PEAK_RIGHT_GRAD_LOG_SCALE = np.array([2.7 * PEAK_RIGHT_ALPHA / (2 * PEAK_VAR**2) * 8.0, 0.0, 0.0])
PEAK_RIGHT_GRAD_DC = PEAK_RIGHT_ALPHA * SH_C0 * np.array([1.0, 1.0, 0.0])


# ------------------------------------------------------------ "jacobian" scene
JAC = dict(fx=100.0, fy=100.0, cx=50.0, cy=40.0, width=100, height=80,
           log_scale=math.log(0.1), lim_x=0.65, lim_y=0.52)
# Camera-space points at depth 2 (identity camera: mean = point).
JAC_MEANS = np.array([
    [2.0, 0.0, -2.0],    # x/d = 1.0   -> xc = 0.65 (clamped)
    [2.0, -1.6, -2.0],   # (1.0, -0.8) -> (0.65, -0.52), both clamped
    [-2.0, 0.0, -2.0],   # x/d = -1.0  -> xc = -0.65 (clamped)
    [0.6, 0.0, -2.0],    # x/d = 0.3, inside
    [0.0, 0.8, -2.0],    # y/d = 0.4, inside
    [0.0, -1.2, -2.0],   # y/d = -0.6 -> yc = -0.52 (clamped)
])
JAC_XC = np.array([0.65, 0.65, -0.65, 0.3, 0.0, 0.0])
JAC_YC = np.array([0.0, -0.52, 0.0, 0.0, 0.4, -0.52])
JAC_X_INSIDE = np.array([False, False, False, True, True, True])
JAC_Y_INSIDE = np.array([True, False, True, True, True, False])


def jac_covariance() -> np.ndarray:
    """[6, 2, 2] screen covariances of the jacobian scene."""
    xc, yc = JAC_XC, JAC_YC
    s00 = 25.0 * (1 + xc * xc) + 0.03
    s01 = -25.0 * xc * yc
    s11 = 25.0 * (1 + yc * yc) + 0.03
    return np.stack((np.stack((s00, s01), -1), np.stack((s01, s11), -1)), -2)


def jac_inverse() -> np.ndarray:
    return np.linalg.inv(jac_covariance())


def jac_grad_inverse_diagonal(axis: int) -> dict[str, np.ndarray]:
    """Gradients of L = inverse_covariance[i, axis, axis] for the Gaussians
    with Sigma01 = 0 (rows 0, 2, 3, 4, 5; row 1 has both ratios clamped).

    There inv_aa = 1 / Sigma_aa, because dinv_aa/dSigma01 = 2 Sigma_bb Sigma01
    / det^2 = 0.  So dL/dtheta = -(dSigma_aa/dtheta) / Sigma_aa^2.  With
    identity rotations, r the camera-space coordinate on this axis
    (x for axis 0, y for axis 1) and rc = clamp(r/d) its clamped ratio:
      Sigma_aa = s_a^2 f^2/d^2 + s2^2 f^2 rc^2/d^2 + 0.03,
      dSigma_aa/dmean_r = 2 s2^2 f^2 rc / d^3 inside the clamp, 0 outside,
      dSigma_aa/dmean_z = -dSigma_aa/dd = 2 (Sigma_aa - 0.03)/d
                          + (2 s2^2 f^2 rc^2 / d^3 inside the clamp),
      dSigma_aa/dlog s_a = 2 s_a^2 f^2 / d^2 = 50,
      dSigma_aa/dlog s2 = 2 s2^2 f^2 rc^2 / d^2 = 50 rc^2.
    Nothing comes from the other mean coordinate, the other in-plane scale or
    the rotation: an isotropic Gaussian does not depend on its rotation.
    """
    rows = np.array([0, 2, 3, 4, 5])
    rc = (JAC_XC if axis == 0 else JAC_YC)[rows]
    inside = (JAC_X_INSIDE if axis == 0 else JAC_Y_INSIDE)[rows]
    d, s2, f = 2.0, 0.01, 100.0
    sig = jac_covariance()[rows, axis, axis]
    ds_dr = np.where(inside, 2 * s2 * f * f * rc / d**3, 0.0)
    ds_dz = 2 * (sig - 0.03) / d + np.where(inside, 2 * s2 * f * f * rc * rc / d**3, 0.0)
    zero = np.zeros_like(rc)
    k = -1.0 / sig**2
    mean = np.stack((ds_dr, zero, ds_dz) if axis == 0 else (zero, ds_dr, ds_dz), -1)
    ls = np.stack((np.full_like(rc, 50.0), zero, 50.0 * rc * rc) if axis == 0
                  else (zero, np.full_like(rc, 50.0), 50.0 * rc * rc), -1)
    return dict(rows=rows, mean=k[:, None] * mean, log_scale=k[:, None] * ls)
