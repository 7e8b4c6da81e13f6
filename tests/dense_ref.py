"""Independent float64 restatement of the rasterizer for small scenes (test infrastructure).

Written in matrix form with torch float64 so that torch.autograd supplies
exact gradients; it shares no code with the C oracle or the HIP kernels.
Each step follows the reference's stated semantics:

* projection and EWA covariance (preprocess_kernels.py:133-269): view depth
  from the row-vector view matrix, homogeneous divide by w + 1e-7, Sigma =
  R diag(s^2) R^T from the unnormalised quaternion (w, x, y, z), camera-space
  x/z and y/z clamped to 1.3 tan(fov) (a clamped coordinate held constant
  in the gradient, as the reference's backward does), cov2D = J W Sigma W^T J^T + 0.3 I,
  conic = cov2D^-1, radius = ceil(3 sqrt(mid + sqrt(max(0.1, mid^2 - det)))),
  pixel = ((ndc + 1) S - 1) / 2, culled when z <= 0.2, |det| <= 1e-7 or the
  3-sigma tile rectangle is empty;
* SH colour (preprocess_kernels.py:272-342): real SH to degree 3 of the
  normalised direction from the camera centre, + 0.5, clamped at 0;
* blending (render_kernels.py:16-147): per pixel, the Gaussians whose tile
  set holds the pixel's tile, in (depth, index) order; power > 0 and
  alpha = min(0.99, o e^power) < 1/255 skipped; the pixel stops, without that
  Gaussian, once T (1 - alpha) < 1e-4; colour + T_final bg; alpha and depth
  are the alpha-T weighted sums.
"""

from __future__ import annotations

import math

import numpy as np
import torch

BLOCK = 16
SH_C0 = 0.28209479177387814
SH_C1 = 0.4886025119029199
SH_C2 = (1.0925484305920792, -1.0925484305920792, 0.31539156525252005, -1.0925484305920792, 0.5462742152960396)
SH_C3 = (-0.5900435899266435, 2.890611442640554, -0.4570457994644658, 0.3731763325901154, -0.4570457994644658,
         1.445305721320277, -0.5900435899266435)


def quat_to_rot(q: torch.Tensor) -> torch.Tensor:
    w, x, y, z = q.unbind(-1)
    return torch.stack([
        torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)], -1),
        torch.stack([2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)], -1),
        torch.stack([2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], -1),
    ], -2)


def covariance_upper(scales: np.ndarray, rotations: np.ndarray, scale_modifier: float = 1.0) -> np.ndarray:
    """(N, 6) upper triangle (xx, xy, xz, yy, yz, zz) of R diag(s^2) R^T in float64."""
    R = quat_to_rot(torch.tensor(np.asarray(rotations), dtype=torch.float64))
    S2 = torch.diag_embed((torch.tensor(np.asarray(scales), dtype=torch.float64) * scale_modifier) ** 2)
    sig = (R @ S2 @ R.transpose(1, 2)).numpy()
    return np.stack([sig[:, 0, 0], sig[:, 0, 1], sig[:, 0, 2], sig[:, 1, 1], sig[:, 1, 2], sig[:, 2, 2]], 1)


def sh_basis(d: torch.Tensor, degree: int) -> torch.Tensor:
    """(N, (degree+1)^2) real SH basis values in the 3DGS sign convention."""
    x, y, z = d.unbind(-1)
    cols = [torch.full_like(x, SH_C0)]
    if degree > 0:
        cols += [-SH_C1 * y, SH_C1 * z, -SH_C1 * x]
    if degree > 1:
        xx, yy, zz = x * x, y * y, z * z
        cols += [SH_C2[0] * x * y, SH_C2[1] * y * z, SH_C2[2] * (2 * zz - xx - yy), SH_C2[3] * x * z,
                 SH_C2[4] * (xx - yy)]
    if degree > 2:
        cols += [SH_C3[0] * y * (3 * xx - yy), SH_C3[1] * x * y * z, SH_C3[2] * y * (4 * zz - xx - yy),
                 SH_C3[3] * z * (2 * zz - 3 * xx - 3 * yy), SH_C3[4] * x * (4 * zz - xx - yy),
                 SH_C3[5] * z * (xx - yy), SH_C3[6] * x * (xx - 3 * yy)]
    return torch.stack(cols, -1)


def tile_rect(px: float, py: float, r: int, gx: int, gy: int):
    def clamp(v, hi):
        return min(hi, max(0, v))
    return (clamp(int((px - r) / BLOCK), gx), clamp(int((py - r) / BLOCK), gy),
            clamp(int((px + r + BLOCK - 1) / BLOCK), gx), clamp(int((py + r + BLOCK - 1) / BLOCK), gy))


def preprocess(means, scales, rots, view, proj, campos, tanfovx, tanfovy, W, H, shs=None, degree=0,
               colors=None, scale_modifier=1.0, cov3d=None, filter_variance=0.0) -> dict:
    """float64 preprocess + colour; tensors keep their autograd history.  With
    cov3d (N, 6: xx, xy, xz, yy, yz, zz) the 3D covariance is taken as given.
    A non-zero filter_variance f is the Mip-Splatting screen-space filter
    (backend_mip_3dgs.py:63-102): Gaussians kept by the base cull get
    cov2D + f I, their conic is its inverse and their radius
    ceil(3 sqrt(lambda_max)) of the filtered covariance (floored at 0.1)."""
    V = view.reshape(16)
    P = proj.reshape(16)
    x, y, z = means.unbind(1)
    vz = V[2] * x + V[6] * y + V[10] * z + V[14]
    hom_x = P[0] * x + P[4] * y + P[8] * z + P[12]
    hom_y = P[1] * x + P[5] * y + P[9] * z + P[13]
    hom_w = P[3] * x + P[7] * y + P[11] * z + P[15]
    inv_w = 1.0 / (hom_w + 1e-7)
    ndc = torch.stack([hom_x * inv_w, hom_y * inv_w], 1)

    Wrot = torch.stack([torch.stack([V[c * 4 + r] for c in range(3)]) for r in range(3)])
    if cov3d is not None:
        c = cov3d
        sigma = torch.stack([torch.stack([c[:, 0], c[:, 1], c[:, 2]], -1),
                             torch.stack([c[:, 1], c[:, 3], c[:, 4]], -1),
                             torch.stack([c[:, 2], c[:, 4], c[:, 5]], -1)], -2)
    else:
        Rm = quat_to_rot(rots)
        S2 = torch.diag_embed((scales * scale_modifier) ** 2)
        sigma = Rm @ S2 @ Rm.transpose(1, 2)
    pv = means @ Wrot.T + torch.stack([V[12], V[13], V[14]])
    fx = W / (2.0 * tanfovx)
    fy = H / (2.0 * tanfovy)
    limx, limy = 1.3 * tanfovx, 1.3 * tanfovy
    # A clamped camera-space coordinate is a constant for the gradient: the
    # reference masks its gradient and differentiates the Jacobian in z as if
    # it were fixed (backward_kernels.py:134-137, 212-214; 827-829).
    rx, ry = pv[:, 0] / vz, pv[:, 1] / vz
    tx = torch.clamp(rx, -limx, limx) * vz
    ty = torch.clamp(ry, -limy, limy) * vz
    tx = torch.where((rx < -limx) | (rx > limx), tx.detach(), tx)
    ty = torch.where((ry < -limy) | (ry > limy), ty.detach(), ty)
    zero = torch.zeros_like(vz)
    J = torch.stack([torch.stack([fx / vz, zero, -fx * tx / (vz * vz)], -1),
                     torch.stack([zero, fy / vz, -fy * ty / (vz * vz)], -1)], -2)
    T = J @ Wrot
    cov = T @ sigma @ T.transpose(1, 2)
    a = cov[:, 0, 0] + 0.3
    b = cov[:, 0, 1]
    c = cov[:, 1, 1] + 0.3
    det = a * c - b * b
    conic = torch.stack([c / det, -b / det, a / det], 1)
    pix = torch.stack([((ndc[:, 0] + 1.0) * W - 1.0) * 0.5, ((ndc[:, 1] + 1.0) * H - 1.0) * 0.5], 1)

    gx, gy = (W + BLOCK - 1) // BLOCK, (H + BLOCK - 1) // BLOCK
    n = means.shape[0]
    radii = np.zeros(n, np.int64)
    ad, cd, dd = a.detach().numpy(), c.detach().numpy(), det.detach().numpy()
    vzd, pixd = vz.detach().numpy(), pix.detach().numpy()
    for i in range(n):
        if vzd[i] <= 0.2 or abs(dd[i]) <= 1e-7:
            continue
        mid = 0.5 * (ad[i] + cd[i])
        lam = mid + math.sqrt(max(0.1, mid * mid - dd[i]))
        r = int(math.ceil(3.0 * math.sqrt(lam)))
        x0, y0, x1, y1 = tile_rect(pixd[i, 0], pixd[i, 1], r, gx, gy)
        if (x1 - x0) * (y1 - y0) > 0:
            radii[i] = r
    if filter_variance != 0.0:
        a = a + filter_variance
        c = c + filter_variance
        det = a * c - b * b
        conic = torch.stack([c / det, -b / det, a / det], 1)
        ad, cd, dd, bd = a.detach().numpy(), c.detach().numpy(), det.detach().numpy(), b.detach().numpy()
        for i in range(n):
            if radii[i] == 0:
                continue
            if not dd[i] > 1e-12:
                radii[i] = 0
                continue
            lam = 0.5 * (ad[i] + cd[i]) + math.sqrt(max(0.25 * (ad[i] - cd[i]) ** 2 + bd[i] ** 2, 0.0))
            radii[i] = int(math.ceil(3.0 * math.sqrt(max(lam, 0.1))))

    if colors is None:
        d = means - campos.reshape(1, 3)
        d = d / torch.sqrt(torch.clamp((d * d).sum(1, keepdim=True), min=1e-20))
        basis = sh_basis(d, degree)
        k = basis.shape[1]
        raw = (basis[:, :, None] * shs[:, :k, :]).sum(1) + 0.5
        clamped = raw < 0.0
        rgb = torch.clamp(raw, min=0.0)
    else:
        rgb = colors
        clamped = torch.zeros_like(colors, dtype=torch.bool)
    return {"depth": vz, "ndc": ndc, "pix": pix, "cov2d": torch.stack([a, b, c], 1), "conic": conic,
            "radii": radii, "rgb": rgb, "clamped": clamped}


def render(pix, conic, opac, rgb, depth, radii, tile_sets, W, H, bg, compute_depth=True, top_k=0):
    """Dense float64 blend; tile_sets[g] is the set of tile ids Gaussian g is binned to."""
    gx = (W + BLOCK - 1) // BLOCK
    ys, xs = torch.meshgrid(torch.arange(H, dtype=torch.float64), torch.arange(W, dtype=torch.float64),
                            indexing="ij")
    tile = (torch.div(ys, BLOCK, rounding_mode="floor") * gx + torch.div(xs, BLOCK, rounding_mode="floor")).long()
    n = pix.shape[0]
    dep = depth.detach().numpy()
    order = [g for g in np.lexsort((np.arange(n), dep)) if radii[g] > 0 and tile_sets[g]]
    # 1-based position of each Gaussian in each tile's list, for n_contrib
    pos_in_tile = {}
    count = {}
    for g in order:
        for t in tile_sets[g]:
            count[t] = count.get(t, 0) + 1
            pos_in_tile[(g, t)] = count[t]
    Tr = torch.ones(H, W, dtype=torch.float64)
    color = torch.zeros(3, H, W, dtype=torch.float64)
    dsum = torch.zeros(H, W, dtype=torch.float64)
    asum = torch.zeros(H, W, dtype=torch.float64)
    done = torch.zeros(H, W, dtype=torch.bool)
    n_contrib = torch.zeros(H, W, dtype=torch.long)
    ids = torch.full((top_k, H, W), -1, dtype=torch.long)
    weights = torch.zeros(top_k, H, W, dtype=torch.float64)
    xmu = torch.zeros(2, top_k, H, W, dtype=torch.float64)
    nsucc = torch.zeros(H, W, dtype=torch.long)
    for g in order:
        in_tile = torch.zeros(H, W, dtype=torch.bool)
        for t in tile_sets[g]:
            in_tile |= tile == t
        dx = pix[g, 0] - xs
        dy = pix[g, 1] - ys
        power = -0.5 * (conic[g, 0] * dx * dx + conic[g, 2] * dy * dy) - conic[g, 1] * dx * dy
        alpha = torch.clamp(opac[g] * torch.exp(power), max=0.99)
        cand = in_tile & ~done & (power <= 0.0) & (alpha >= 1.0 / 255.0)
        test_T = Tr * (1.0 - alpha)
        stop = cand & (test_T < 1e-4)
        done = done | stop
        blend = cand & ~stop
        w = alpha * Tr
        color = color + torch.where(blend[None], rgb[g][:, None, None] * w[None], 0.0)
        asum = asum + torch.where(blend, w, 0.0)
        if compute_depth:
            dsum = dsum + torch.where(blend, depth[g] * w, 0.0)
        if top_k:
            sel = blend & (nsucc < top_k)
            if bool(sel.any()):
                yy, xx = torch.nonzero(sel, as_tuple=True)
                k = nsucc[yy, xx]
                ids[k, yy, xx] = g
                weights = weights.index_put((k, yy, xx), w[yy, xx])
                xmu = xmu.index_put((torch.zeros_like(k), k, yy, xx), dx[yy, xx])
                xmu = xmu.index_put((torch.ones_like(k), k, yy, xx), dy[yy, xx])
            nsucc = nsucc + blend.long()
        if bool(blend.any()):
            yy, xx = torch.nonzero(blend, as_tuple=True)
            n_contrib[yy, xx] = torch.tensor([pos_in_tile[(g, int(t))] for t in tile[yy, xx]], dtype=torch.long)
        Tr = torch.where(blend, test_T, Tr)
    color = color + Tr[None] * bg.reshape(3, 1, 1)
    out = {"color": color, "alpha": asum[None], "depth": dsum[None], "n_contrib": n_contrib}
    if top_k:
        out.update(ids=ids, weights=weights, x_mu=xmu)
    return out
