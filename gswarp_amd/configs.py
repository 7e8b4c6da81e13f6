"""Synthetic scenes and cameras for the benchmark configurations.

Camera convention (the one the reference kernels read, e.g.
gswarp/_internal/backends/warp/preprocess_kernels.py:134-146):
``viewmatrix`` is the world->camera matrix transposed (row-vector layout,
camera looking down +z with y pointing down), and ``projmatrix`` is
``viewmatrix @ P^T`` where P is the usual OpenGL-style perspective matrix
with z mapped by zfar/(zfar-znear).  ``campos`` is the camera centre in world
space.

Configurations (all inputs fp32, drawn on the CPU from one
``torch.Generator().manual_seed(seed)`` in this order: means, log-scales,
quaternions, opacity logits, SH DC, SH rest; then moved to the device):

  0  10,000 Gaussians, 256x256, SH degree 0, forward only.  Means x,y ~ U[-1,1],
     z ~ U[2,6] in camera space with an identity view; log-scales ~ N(-4.5, 0.5);
     rotations uniform on S^3 (normalised 4-D normal draws, [w,x,y,z]);
     opacity = sigmoid(N(0,1)); DC ~ N(0, 0.3).  FoV 60 deg both axes.
  1  100,000 Gaussians, 800x800, SH degree 3 (DC ~ N(0,0.3), bands 1-3 ~ N(0,0.05)),
     config-0 distributions in world space; camera at (0,0,-4) looking at the
     origin, FoV 50 deg.  dL/dcolor ~ N(0,1); dL/ddepth = dL/dalpha = 0.
  2  1,000,000 Gaussians, 1920x1080, SH degree 3; means ~ N(0, diag(3,1.5,3));
     log-scales ~ N(-5, 0.7); camera on a sphere of radius 6 looking at the
     origin, direction drawn per iteration from seed*1000003+iteration;
     FoVx = 60 deg, FoVy = 2 atan(tan 30 deg * H / W).  Upstream gradients
     ~ N(0,1) on colour, depth and alpha.
  3  As 2 with 5,000,000 Gaussians; log-scales from a 90/10 mixture of
     N(-5.5, 0.5) and N(-2, 0.5) (both component draws are made, then a U[0,1)
     draw per Gaussian selects the second when < 0.1); opacity = sigmoid(N(1,1)).
  4  Flow API: 1,000,000 Gaussians, 1280x720, SH degree 3, distributions as 2;
     top-K = 20; upstream gradient ~ N(0,1) on colour and on x_mu.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

ZNEAR = 0.01
ZFAR = 100.0


@dataclass(frozen=True)
class ConfigSpec:
    index: int
    count: int
    width: int
    height: int
    sh_degree: int
    backward: bool
    flow: bool = False
    description: str = ""


CONFIGS = {
    0: ConfigSpec(0, 10_000, 256, 256, 0, False, description="10k, 256x256, SH0, forward only"),
    1: ConfigSpec(1, 100_000, 800, 800, 3, True, description="100k, 800x800, SH3, fwd+bwd"),
    2: ConfigSpec(2, 1_000_000, 1920, 1080, 3, True, description="1M, 1920x1080, SH3, fwd+bwd, depth+alpha"),
    3: ConfigSpec(3, 5_000_000, 1920, 1080, 3, True, description="5M heavy-overlap mixture, 1920x1080, SH3"),
    4: ConfigSpec(4, 1_000_000, 1280, 720, 3, True, flow=True, description="flow API, 1M, 1280x720, SH3, K=20"),
}


def projection_matrix(znear: float, zfar: float, fovx: float, fovy: float) -> torch.Tensor:
    """Perspective matrix (column-vector convention) for symmetric frusta."""
    tan_x = math.tan(fovx / 2.0)
    tan_y = math.tan(fovy / 2.0)
    top, right = tan_y * znear, tan_x * znear
    P = torch.zeros(4, 4, dtype=torch.float64)
    P[0, 0] = 2.0 * znear / (2.0 * right)
    P[1, 1] = 2.0 * znear / (2.0 * top)
    P[3, 2] = 1.0
    P[2, 2] = zfar / (zfar - znear)
    P[2, 3] = -(zfar * znear) / (zfar - znear)
    return P


def look_at(position, target=(0.0, 0.0, 0.0), up=(0.0, 1.0, 0.0)) -> torch.Tensor:
    """World->camera matrix (column-vector convention): x right, y down, z forward."""
    c = torch.tensor(position, dtype=torch.float64)
    f = torch.tensor(target, dtype=torch.float64) - c
    f = f / f.norm()
    u = torch.tensor(up, dtype=torch.float64)
    if torch.cross(f, u, dim=0).norm() < 1e-6:
        u = torch.tensor((0.0, 0.0, 1.0), dtype=torch.float64)
    x = torch.cross(f, u, dim=0)
    x = x / x.norm()
    y = torch.cross(f, x, dim=0)
    R = torch.stack([x, y, f])
    W2C = torch.eye(4, dtype=torch.float64)
    W2C[:3, :3] = R
    W2C[:3, 3] = -R @ c
    return W2C


def camera(width: int, height: int, fovx: float, fovy: float, world_to_camera: torch.Tensor) -> dict:
    """Rasterizer camera fields from a world->camera matrix (float64 in, fp32 out)."""
    view = world_to_camera.T.contiguous()
    proj = projection_matrix(ZNEAR, ZFAR, fovx, fovy).T.contiguous()
    full = view @ proj
    cam_center = torch.linalg.inv(world_to_camera)[:3, 3]
    return {
        "width": width,
        "height": height,
        "tanfovx": math.tan(fovx * 0.5),
        "tanfovy": math.tan(fovy * 0.5),
        "viewmatrix": view.to(torch.float32),
        "projmatrix": full.to(torch.float32),
        "campos": cam_center.to(torch.float32),
    }


def _random_quaternions(g: torch.Generator, n: int) -> torch.Tensor:
    q = torch.randn(n, 4, generator=g)
    return q / q.norm(dim=1, keepdim=True)


def _sh_coefficients(g: torch.Generator, n: int, degree: int) -> torch.Tensor:
    dc = torch.randn(n, 1, 3, generator=g) * 0.3
    k = (degree + 1) ** 2
    if k == 1:
        return dc
    rest = torch.randn(n, k - 1, 3, generator=g) * 0.05
    return torch.cat([dc, rest], dim=1)


def orbit_camera(spec: ConfigSpec, seed: int, iteration: int, radius: float = 6.0) -> dict:
    g = torch.Generator().manual_seed(seed * 1_000_003 + iteration)
    d = torch.randn(3, generator=g, dtype=torch.float64)
    d = d / d.norm()
    fovx = math.radians(60.0)
    fovy = 2.0 * math.atan(math.tan(fovx / 2.0) * spec.height / spec.width)
    return camera(spec.width, spec.height, fovx, fovy, look_at(tuple((radius * d).tolist())))


def make_scene(config: int, *, seed: int = 0, iteration: int = 0, count: int | None = None,
               width: int | None = None, height: int | None = None, device: str | torch.device = "cpu") -> dict:
    """Inputs of one benchmark configuration as a dict of tensors and scalars.

    ``count``/``width``/``height`` shrink a configuration for parity tests
    while keeping its distributions and camera construction.
    """
    base = CONFIGS[config]
    spec = ConfigSpec(base.index, count or base.count, width or base.width, height or base.height, base.sh_degree,
                      base.backward, base.flow, base.description)
    n = spec.count
    g = torch.Generator().manual_seed(seed)
    if config in (0, 1):
        means = torch.empty(n, 3)
        means[:, 0].uniform_(-1.0, 1.0, generator=g)
        means[:, 1].uniform_(-1.0, 1.0, generator=g)
        means[:, 2].uniform_(2.0, 6.0, generator=g)
        log_scales = torch.randn(n, 3, generator=g) * 0.5 - 4.5
    else:
        means = torch.randn(n, 3, generator=g) * torch.tensor([math.sqrt(3.0), math.sqrt(1.5), math.sqrt(3.0)])
        if config == 3:
            small = torch.randn(n, 3, generator=g) * 0.5 - 5.5
            large = torch.randn(n, 3, generator=g) * 0.5 - 2.0
            pick = torch.rand(n, generator=g) < 0.1
            log_scales = torch.where(pick[:, None], large, small)
        else:
            log_scales = torch.randn(n, 3, generator=g) * 0.7 - 5.0
    rotations = _random_quaternions(g, n)
    logits = torch.randn(n, 1, generator=g) + (1.0 if config == 3 else 0.0)
    opacities = torch.sigmoid(logits)
    shs = _sh_coefficients(g, n, spec.sh_degree)

    if config == 0:
        fov = math.radians(60.0)
        cam = camera(spec.width, spec.height, fov, fov, torch.eye(4, dtype=torch.float64))
    elif config == 1:
        fov = math.radians(50.0)
        cam = camera(spec.width, spec.height, fov, fov, look_at((0.0, 0.0, -4.0)))
    else:
        cam = orbit_camera(spec, seed, iteration)

    scene = {
        "config": config,
        "spec": spec,
        "means3D": means,
        "scales": torch.exp(log_scales),
        "rotations": rotations,
        "opacities": opacities,
        "shs": shs,
        "sh_degree": spec.sh_degree,
        "bg": torch.zeros(3),
        "scale_modifier": 1.0,
        **cam,
    }
    for key, value in list(scene.items()):
        if isinstance(value, torch.Tensor):
            scene[key] = value.to(device=device, dtype=torch.float32).contiguous()
    return scene


def upstream_gradients(config: int, width: int, height: int, *, seed: int = 0, top_k: int = 20,
                       device: str | torch.device = "cpu") -> dict:
    """Upstream gradients of the benchmark loss for one configuration."""
    g = torch.Generator().manual_seed(seed + 7919)
    grads = {"color": torch.randn(3, height, width, generator=g)}
    if config in (2, 3):
        grads["depth"] = torch.randn(1, height, width, generator=g)
        grads["alpha"] = torch.randn(1, height, width, generator=g)
    else:
        grads["depth"] = torch.zeros(1, height, width)
        grads["alpha"] = torch.zeros(1, height, width)
    if config == 4:
        grads["x_mu"] = torch.randn(2, top_k, height, width, generator=g)
    return {k: v.to(device=device, dtype=torch.float32).contiguous() for k, v in grads.items()}


def scene_to_numpy(scene: dict) -> dict:
    """Host copies (numpy) of a scene, for the CPU oracle."""
    out = {}
    for key, value in scene.items():
        if isinstance(value, torch.Tensor):
            out[key] = value.detach().cpu().numpy()
        else:
            out[key] = value
    out["shs"] = out["shs"] if "shs" in out else None
    return out
