"""Receptive-field geometry for the LUT layers, backed by the native builder
(spiky_grow_cuboid in libspiky_lut.so).

Mirrors the public helpers of the reference's src/spiky/util/synapse_growth.py:
GrowthCommand, PointSamplingType / PointSamplingPolicy, sample_random_points,
sample_grid_points, Conv2DSynapseGrowthHelper (:364-449),
RandomRectanglesSynapseGrowthHelper (:531-643) and
GivenRectanglesSynapseGrowthHelper (:646-703).  Each helper returns a
ChunkOfConnections in the reference's buffer format.  Neuron coordinates,
cuboid bounds and group-centre sampling follow the reference line by line in
meaning: a source at (x, y, z) connects to targets inside
[x+x1, x+x2] x [y+y1, y+y2] x [z+z1, z+z2] (fp32 bounds).
"""
import ctypes
from dataclasses import dataclass
from enum import Enum

import numpy as np
import torch

from .. import _native
from .chunk_of_connections import build_connections


@dataclass(frozen=True, order=True)
class GrowthCommand:
    """Cuboid growth rule (reference synapse_growth.py:11-55)."""
    target_type: int
    synapse_meta_index: int
    x1: float
    y1: float
    z1: float
    x2: float
    y2: float
    z2: float
    p: float = 1.0
    max_synapses: int = 0

    def __post_init__(self):
        assert 0 <= self.target_type
        assert 0 <= self.synapse_meta_index
        assert self.x1 < self.x2
        assert self.y1 < self.y2
        assert self.z1 < self.z2
        assert 0 < self.p <= 1.0
        assert self.max_synapses >= 0


def grow_cuboid(src_ids, src_xyz, tgt_ids, tgt_xyz, command: GrowthCommand, seed=None,
                max_per_source=0):
    """Runs one growth command natively.  Returns (sorted source ids, offsets, targets)."""
    src_ids = np.ascontiguousarray(np.asarray(src_ids, dtype=np.int64).reshape(-1)).astype(np.int32)
    tgt_ids = np.ascontiguousarray(np.asarray(tgt_ids, dtype=np.int64).reshape(-1)).astype(np.int32)
    src_xyz = np.ascontiguousarray(np.asarray(src_xyz, dtype=np.float32).reshape(-1, 3))
    tgt_xyz = np.ascontiguousarray(np.asarray(tgt_xyz, dtype=np.float32).reshape(-1, 3))
    order = np.argsort(src_ids, kind="stable")
    src_ids, src_xyz = np.ascontiguousarray(src_ids[order]), np.ascontiguousarray(src_xyz[order])
    cub = np.array([command.x1, command.y1, command.z1, command.x2, command.y2, command.z2],
                   dtype=np.float32)
    offs = np.zeros(src_ids.size + 1, dtype=np.int64)
    total = ctypes.c_uint64()
    L = _native.lib()
    vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    seed_v = 0 if seed is None else int(seed) & 0xFFFFFFFFFFFFFFFF
    _native.check(L.spiky_grow_cuboid(src_ids.size, vp(src_ids), vp(src_xyz), tgt_ids.size,
                                      vp(tgt_ids), vp(tgt_xyz), vp(cub), float(command.p), seed_v,
                                      int(max_per_source), vp(offs), None, 0, ctypes.byref(total)))
    tg = np.zeros(max(int(total.value), 1), dtype=np.int32)
    _native.check(L.spiky_grow_cuboid(src_ids.size, vp(src_ids), vp(src_xyz), tgt_ids.size,
                                      vp(tgt_ids), vp(tgt_xyz), vp(cub), float(command.p), seed_v,
                                      int(max_per_source), vp(offs), vp(tg), tg.size,
                                      ctypes.byref(total)))
    return src_ids, offs, tg[:int(total.value)]


def sample_random_points(n_points, ow, oh, clamp_x, clamp_y, is_normal=False, mu=None, sigma=None,
                         seed=None, device=None):
    """(x, y) points in [0,ow]x[0,oh] (reference synapse_growth.py:452-484),
    drawn with the same torch calls in the same order."""
    device = device or "cpu"
    ow = float(ow)
    oh = float(oh)
    gen = torch.Generator(device=device)
    if seed is not None:
        gen.manual_seed(seed)
    if is_normal:
        if mu is None:
            mu = (ow / 2.0, oh / 2.0)
        if sigma is None:
            sigma = (ow / 6.0, oh / 6.0)
        mx, my = mu
        sx, sy = sigma
        x = torch.randn(n_points, device=device, generator=gen) * sx + mx
        y = torch.randn(n_points, device=device, generator=gen) * sy + my
        return torch.stack([x.clamp(*clamp_x), y.clamp(*clamp_y)], dim=1)
    x = torch.rand(n_points, device=device, generator=gen) * ow
    y = torch.rand(n_points, device=device, generator=gen) * oh
    return torch.stack([x.clamp(*clamp_x), y.clamp(*clamp_y)], dim=1)


def sample_grid_points(gw, gh, center_x, center_y, stride_x, stride_y, device):
    """Regular grid of points, row-major (reference synapse_growth.py:487-497)."""
    xs = center_x + stride_x * torch.arange(gw, device=device, dtype=torch.float32)
    ys = center_y + stride_y * torch.arange(gh, device=device, dtype=torch.float32)
    yy, xx = torch.meshgrid(ys, xs, indexing="ij")
    return torch.stack([xx.reshape(-1), yy.reshape(-1)], dim=1)


class PointSamplingType(Enum):
    RandomUniform = 0
    RandomNormal = 1
    Grid = 2


@dataclass(frozen=True)
class PointSamplingPolicy:
    type: PointSamplingType
    mu: float = None
    sigma: float = None
    pad_h: float = 0.0
    pad_w: float = 0.0
    grid_h: int = None
    grid_w: int = None
    stride_h: int = None
    stride_w: int = None

    def __post_init__(self):
        if self.sigma is not None:
            assert self.sigma > 0.0
        assert self.pad_h >= 0.0
        assert self.pad_w >= 0.0
        if self.grid_h is not None:
            assert self.grid_h > 0
        if self.grid_w is not None:
            assert self.grid_w > 0
        if self.stride_h is not None:
            assert self.stride_h >= 0
        if self.stride_w is not None:
            assert self.stride_w >= 0


def _window_command(rw, rh, p):
    # a window of rw x rh cells centred on the target: +-((r-1)/2 + 1e-4)
    return GrowthCommand(target_type=1, synapse_meta_index=0,
                         x1=-((rw - 1) / 2) - 1e-4, y1=-((rh - 1) / 2) - 1e-4, z1=0.5,
                         x2=((rw - 1) / 2) + 1e-4, y2=((rh - 1) / 2) + 1e-4, z2=1.5, p=p)


class Conv2DSynapseGrowthHelper(object):
    """Sliding-window receptive fields (reference synapse_growth.py:364-449)."""

    def __init__(self, h, w, rh, rw, sh, sw, kh, kw, p=1.0, n_input_channels=None):
        self.h, self.w, self.rw, self.rh, self.sw, self.sh = h, w, rw, rh, sw, sh
        self.kw, self.kh, self.p = kw, kh, p
        self.n_input_channels = n_input_channels
        self.num_win_h = ((self.h - self.rh) // self.sh) + 1
        self.num_win_w = ((self.w - self.rw) // self.sw) + 1
        self.out_h = self.num_win_h * self.kh
        self.out_w = self.num_win_w * self.kw

    def output_coords(self):
        out = np.zeros((self.out_h * self.out_w, 3), dtype=np.float32)
        for win_y in range(self.num_win_h):
            for win_x in range(self.num_win_w):
                cy = win_y * self.sh + ((self.rh - 1) / 2)
                cx = win_x * self.sw + ((self.rw - 1) / 2)
                for by in range(self.kh):
                    for bx in range(self.kw):
                        k = (win_y * self.kh + by) * self.out_w + win_x * self.kw + bx
                        out[k] = (cx, cy, 1.0)
        return out

    def input_coords(self, n_ch):
        ys, xs = np.meshgrid(np.arange(self.h), np.arange(self.w), indexing="ij")
        xy = np.stack([xs.reshape(-1), ys.reshape(-1), np.zeros(self.h * self.w)], 1)
        return np.repeat(xy, n_ch, axis=0).astype(np.float32)

    def grow_synapses(self, input_ids, output_ids, device=None, synapse_group_size=64,
                      max_groups_in_buffer=2 ** 20, seed=None):
        n_ch = 1 if self.n_input_channels is None else self.n_input_channels
        assert tuple(input_ids.shape) == ((self.h, self.w) if self.n_input_channels is None
                                          else (self.h, self.w, n_ch))
        assert tuple(output_ids.shape) == (self.out_h, self.out_w)
        assert bool((input_ids > 0).all()) and bool((output_ids > 0).all())
        src, offs, tg = grow_cuboid(input_ids.reshape(-1).cpu().numpy(), self.input_coords(n_ch),
                                    output_ids.reshape(-1).cpu().numpy(), self.output_coords(),
                                    _window_command(self.rw, self.rh, self.p), seed)
        return build_connections(src, offs, tg, synapse_group_size, 0, device)

    def n_connections(self):
        return self.num_win_h * self.num_win_w * self.kh * self.kw * self.rh * self.rw


class RandomRectanglesSynapseGrowthHelper(object):
    """Detector groups at sampled centres, each reading an rh x rw window of
    the input grid (reference synapse_growth.py:531-643)."""

    def __init__(self, h, w, rh, rw, oh, ow, n_outputs, p=1.0, n_out_channels=1,
                 input_sparsity_mask=None,
                 output_sampling_policy: PointSamplingPolicy = PointSamplingPolicy(PointSamplingType.RandomUniform)):
        assert w > 0 and h > 0 and rw > 0 and rh > 0 and oh > 0 and ow > 0
        assert 0.0 < p <= 1.0
        assert n_outputs > 0 and n_out_channels > 0
        assert output_sampling_policy is not None
        self.h, self.w, self.rw, self.rh, self.ow, self.oh = h, w, rw, rh, ow, oh
        self.p = p
        self.n_out_channels = n_out_channels
        self.n_outputs = n_outputs
        self.input_sparsity_mask = input_sparsity_mask
        self.output_sampling_policy = output_sampling_policy

    def sample_centers(self, seed=None, device=None):
        pol = self.output_sampling_policy
        if pol.type == PointSamplingType.RandomUniform:
            c = sample_random_points(self.n_outputs, self.ow, self.oh, (pol.pad_w, self.w - pol.pad_w),
                                     (pol.pad_h, self.h - pol.pad_h), seed=seed, device=device)
        elif pol.type == PointSamplingType.RandomNormal:
            c = sample_random_points(self.n_outputs, self.ow, self.oh, (pol.pad_w, self.w - pol.pad_w),
                                     (pol.pad_h, self.h - pol.pad_h), is_normal=True, mu=pol.mu,
                                     sigma=pol.sigma, seed=seed, device=device)
        else:
            assert pol.grid_h is not None and pol.grid_w is not None
            assert pol.grid_h * pol.grid_w == self.n_outputs
            c = sample_grid_points(pol.grid_w, pol.grid_h, pol.pad_w, pol.pad_h, pol.stride_w,
                                   pol.stride_h, device=device)
        if self.n_out_channels > 1:
            c = c.view(self.n_outputs, 1, 2).repeat(1, self.n_out_channels, 1).view(
                self.n_outputs * self.n_out_channels, 2)
        return c

    def grow_synapses(self, input_ids, output_ids, device=None, synapse_group_size=64,
                      max_groups_in_buffer=2 ** 20, seed=None):
        assert tuple(input_ids.shape) == (self.h, self.w)
        assert tuple(output_ids.shape) == (self.n_outputs * self.n_out_channels,)
        assert bool((input_ids > 0).all()) and bool((output_ids > 0).all())
        in_xyz = np.zeros((self.h * self.w, 3), dtype=np.float32)
        for y in range(self.h):
            for x in range(self.w):
                m = self.input_sparsity_mask is None or bool(self.input_sparsity_mask[y, x])
                in_xyz[y * self.w + x] = (x, y, 0) if m else (1e30, 1e30, 0)
        centers = self.sample_centers(seed=seed, device="cpu")
        out_xyz = np.ones((self.n_outputs * self.n_out_channels, 3), dtype=np.float32)
        out_xyz[:, :2] = centers.numpy()
        src, offs, tg = grow_cuboid(input_ids.reshape(-1).cpu().numpy(), in_xyz,
                                    output_ids.reshape(-1).cpu().numpy(), out_xyz,
                                    _window_command(self.rw, self.rh, self.p), seed)
        chunk = build_connections(src, offs, tg, synapse_group_size, 0, device)
        return chunk, centers.to(device) if device is not None else centers


class GivenRectanglesSynapseGrowthHelper(object):
    """Projection of given centres onto an output grid: every output cell within
    +-(r/2 + 1e-4) of a centre (reference synapse_growth.py:646-703)."""

    def __init__(self, centers, rh, rw, oh, ow, p=1.0, max_synapses_per_input=None,
                 output_sparsity_mask=None):
        self.centers = centers
        self.rw, self.rh, self.ow, self.oh = rw, rh, ow, oh
        self.p = p
        self.max_synapses_per_input = max_synapses_per_input
        self.output_sparsity_mask = output_sparsity_mask

    def grow_synapses(self, input_ids, output_ids, device=None, synapse_group_size=64,
                      max_groups_in_buffer=2 ** 20, seed=None):
        assert tuple(input_ids.shape) == (self.centers.shape[0],)
        assert tuple(output_ids.shape) == (self.oh, self.ow)
        assert bool((input_ids > 0).all()) and bool((output_ids > 0).all())
        cmd = GrowthCommand(target_type=1, synapse_meta_index=0,
                            x1=-(self.rw / 2) - 1e-4, y1=-(self.rh / 2) - 1e-4, z1=0.5,
                            x2=(self.rw / 2) + 1e-4, y2=(self.rh / 2) + 1e-4, z2=1.5, p=self.p)
        in_xyz = np.zeros((self.centers.shape[0], 3), dtype=np.float32)
        in_xyz[:, :2] = self.centers.detach().cpu().numpy()
        out_xyz = np.zeros((self.oh * self.ow, 3), dtype=np.float32)
        for y in range(self.oh):
            for x in range(self.ow):
                m = self.output_sparsity_mask is None or bool(self.output_sparsity_mask[y, x])
                out_xyz[y * self.ow + x] = (x, y, 1) if m else (1e30, 1e30, 1)
        max_per = self.oh * self.ow if self.max_synapses_per_input is None else self.max_synapses_per_input
        src, offs, tg = grow_cuboid(input_ids.reshape(-1).cpu().numpy(), in_xyz,
                                    output_ids.reshape(-1).cpu().numpy(), out_xyz, cmd, seed,
                                    max_per_source=max_per)
        return build_connections(src, offs, tg, synapse_group_size, 0, device)
