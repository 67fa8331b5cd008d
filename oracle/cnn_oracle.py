"""CPU restatement of 2-D (spatial) plans — TEST INFRASTRUCTURE ONLY.

Only tests/ use this module, as the checker.  Tensors are fp16 arrays [frames][C][H][W]; each
function computes in float64 and rounds once to fp16 where the device stores a tensor.  The
operations are the textbook ones the reference compiles into waves and spatial commands:

  conv2d     wavec.py add_conv2d / k44_wave_compiler.hpp emit_conv_waves (3x3 "same" taps,
             stride 2 through the polyphase S2D scratch, 1x1): y = act(conv(x, w) + b) [+ res]
  maxpool2   kernels/common/kernel44_valu_pack.cuh:30-38 (2x2, stride 2)
  maxpool5   kernel44_valu_pack.cuh:40-55 (5x5, stride 1, padding ignored in the max)
  upsample2  kernel44_valu_pack.cuh:56-64 (nearest)
  upconv2x2  transposed 2x2 convolution, stride 2 (k44_wave_compiler.hpp emit_deconv_waves +
             kernel44_valu_pack.cuh:93-103): y[c][2y+a][2x+b] = b[c] + sum_i w[c][i][a][b] x[i][y][x]
  Layout2D   the padded-plane tensor layout of k44_plan_types.hpp:447-569 (K44ResDesc::init, 2-D
             modes), used to place inputs on and read outputs from the canvas.
Pinned in tests/test_cnn_oracle.py against direct loops, closed forms and scipy/numpy routines.
"""
from dataclasses import dataclass

import numpy as np
from scipy.special import erf

F16 = np.float16


def act(v: np.ndarray, name) -> np.ndarray:
    """Activations of the wave epilogue (orc_act in wave_oracle.c), float64."""
    if name in (None, "none"):
        return v
    if name == "relu":
        return np.maximum(v, 0.0)
    if name == "sigmoid":
        return 1.0 / (1.0 + np.exp(-v))
    if name == "silu":
        return v / (1.0 + np.exp(-v))
    if name == "leaky_relu":
        return np.where(v > 0.1 * v, v, 0.1 * v)
    if name == "gelu":
        return 0.5 * v * (1.0 + erf(v * 0.70710678118654752440))
    raise ValueError(name)


def conv2d_f64(x: np.ndarray, w: np.ndarray, b, stride: int, pad: int, act_name=None,
               res=None) -> np.ndarray:
    """x [F][Cin][H][W] fp16, w [Cout][Cin][kh][kw] fp16 -> float64 [F][Cout][Ho][Wo]."""
    F, C, H, W = x.shape
    Co, Ci, kh, kw = w.shape
    assert Ci == C
    xp = np.zeros((F, C, H + 2 * pad, W + 2 * pad))
    xp[:, :, pad:pad + H, pad:pad + W] = x.astype(np.float64)
    Ho = (H + 2 * pad - kh) // stride + 1
    Wo = (W + 2 * pad - kw) // stride + 1
    wf = w.astype(np.float64)
    out = np.zeros((F, Co, Ho, Wo))
    for ky in range(kh):
        for kx in range(kw):
            win = xp[:, :, ky:ky + stride * (Ho - 1) + 1:stride, kx:kx + stride * (Wo - 1) + 1:stride]
            out += np.einsum("oc,fchw->fohw", wf[:, :, ky, kx], win)
    if b is not None:
        out += b.astype(np.float64)[None, :, None, None]
    out = act(out, act_name)
    if res is not None:
        out = out + res.astype(np.float64)
    return out


def maxpool2(x: np.ndarray) -> np.ndarray:
    F, C, H, W = x.shape
    v = x[:, :, :H // 2 * 2, :W // 2 * 2].reshape(F, C, H // 2, 2, W // 2, 2)
    return v.max(axis=(3, 5))


def maxpool5(x: np.ndarray) -> np.ndarray:
    F, C, H, W = x.shape
    xp = np.full((F, C, H + 4, W + 4), -np.inf, dtype=np.float32)
    xp[:, :, 2:2 + H, 2:2 + W] = x
    out = np.full((F, C, H, W), -np.inf, dtype=np.float32)
    for dy in range(5):
        for dx in range(5):
            out = np.maximum(out, xp[:, :, dy:dy + H, dx:dx + W])
    return out.astype(F16)


def upsample2(x: np.ndarray) -> np.ndarray:
    return x.repeat(2, axis=2).repeat(2, axis=3)


def upconv2x2_f64(x: np.ndarray, w: np.ndarray, b) -> np.ndarray:
    """x [F][Cin][H][W], w [Cout][Cin][2][2] -> float64 [F][Cout][2H][2W]."""
    F, C, H, W = x.shape
    Co = w.shape[0]
    out = np.zeros((F, Co, 2 * H, 2 * W))
    xf = x.astype(np.float64)
    for a in range(2):
        for bb in range(2):
            out[:, :, a::2, bb::2] = np.einsum("oc,fchw->fohw", w[:, :, a, bb].astype(np.float64), xf)
    if b is not None:
        out += b.astype(np.float64)[None, :, None, None]
    return out


@dataclass
class Layout2D:
    """Padded-plane layout of a 2-D tensor (K44ResDesc::init).  tok64: the 64-frame interleaved
    image layout (k44_plan_types.hpp:576-598): pixel (y, x) of frame f at c*channel_stride +
    (f//64)*64*single_stride + ((y+1)*W_pad + x+1)*64 + f%64, frames a multiple of 64 (64-frame
    blocks 64*single_stride apart)."""
    H: int
    W: int
    frames: int = 1
    tok64: bool = False

    @property
    def aligned(self) -> bool:
        return self.W % 64 == 0

    @property
    def W_pad(self) -> int:
        return self.W + 8 if self.aligned else self.W + 4

    @property
    def single_stride(self) -> int:
        if self.aligned:
            return (self.H + 2) * self.W_pad
        tiles = (self.H * self.W_pad + 63) // 64
        return (2 * self.W_pad + tiles * 64 + 63) & ~63

    @property
    def channel_stride(self) -> int:
        return self.frames * self.single_stride

    def offsets(self, C: int) -> np.ndarray:
        """[frames][C][H][W] canvas element offsets relative to the tensor base."""
        f = np.arange(self.frames)[:, None, None, None]
        c = np.arange(C)[None, :, None, None]
        y = np.arange(self.H)[None, None, :, None]
        x = np.arange(self.W)[None, None, None, :]
        if self.tok64:
            assert self.frames % 64 == 0
            return (c * self.channel_stride + (f // 64) * 64 * self.single_stride
                    + ((y + 1) * self.W_pad + x + 1) * 64 + f % 64)
        return (c * self.channel_stride + f * self.single_stride + (y + 1) * self.W_pad + 4 + x)
