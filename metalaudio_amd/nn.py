"""Python mirror of the reference's MetalNN layer API over the C ABI (include/mnn.h).

Names and argument meanings follow Sources/MetalNN (Conv1D.swift, DynamicConv1D.swift,
Normalization.swift, Activations.swift, Linear.swift, Attention.swift, Transformer.swift,
UNet.swift, Model.swift); errors surface as MNNError carrying the mnn_status code that stands in
for the reference's MetalAudioError / SequentialModelError cases. All compute runs in
libmnn.so's HIP kernels; this module only marshals arguments.
"""
from __future__ import annotations

import ctypes as C
from typing import Iterable, Optional, Sequence

import numpy as np

from . import _lib
from ._lib import (ACT, PAD, PRECISION, Conv1dDesc, Conv2dDesc, ConvTranspose1dDesc,
                   ConvTranspose2dDesc, DecoderBlockDesc, EncoderBlockDesc, FreqBlockDesc, MNNError,
                   SeparatorDesc, check, dims, lib)

__all__ = [
    "MNNError", "AudioDevice", "Stream", "Tensor", "Layer", "Conv1D", "DynamicConv1D",
    "FusedConv1D", "GroupNorm", "LayerNorm", "GELU", "GLU", "Linear", "FusedLinear",
    "MultiHeadAttention", "CrossAttention",
    "FeedForward", "UNetEncoderBlock", "ConvTranspose1D", "DynamicConvTranspose1D",
    "UNetDecoderBlock", "unet_padding", "unet_bottleneck_length", "TransformerLayer",
    "CrossTransformerEncoder", "Sequential", "SafeTensors", "BinaryModelFile", "WeightNameMapper",
    "Conv2D", "DynamicConv2D", "ConvTranspose2D", "DynamicConvTranspose2D",
    "FreqUNetEncoderBlock2D", "FreqUNetDecoderBlock2D", "unet_padding_2d", "unet_bottleneck_2d",
    "STFT", "WINDOWS", "Separator", "STEM_NAMES",
    "mfma_probe", "MetalNNCrossTransformerEncoder",
]


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


class AudioDevice:
    """A HIP device (AudioDevice.swift:323-348)."""

    def __init__(self, ordinal: int = 0):
        h = C.c_void_p()
        check(lib().mnn_device_create(ordinal, C.byref(h)))
        self.handle = h
        self._default_stream = None

    @property
    def name(self) -> str:
        buf = C.create_string_buffer(256)
        check(lib().mnn_device_name(self.handle, buf, 256))
        return buf.value.decode()

    def synchronize(self) -> None:
        check(lib().mnn_device_synchronize(self.handle))

    def mark_lost(self) -> None:
        check(lib().mnn_device_mark_lost(self.handle))

    def check_available(self, timeout_ms: int = 1000) -> None:
        check(lib().mnn_device_check_available(self.handle, timeout_ms))

    def set_kernel_timing(self, enable: bool) -> None:
        check(lib().mnn_device_set_kernel_timing(self.handle, int(bool(enable))))

    def kernel_timing(self, substr: str = "") -> tuple[int, float]:
        """(launches, total ms) of timed kernels whose name contains `substr`."""
        n = C.c_int64()
        ms = C.c_double()
        check(lib().mnn_device_kernel_timing(self.handle, substr.encode(), C.byref(n), C.byref(ms)))
        return n.value, ms.value

    def reset_kernel_timing(self) -> None:
        check(lib().mnn_device_reset_kernel_timing(self.handle))

    def close(self) -> None:
        if self.handle:
            check(lib().mnn_device_destroy(self.handle))
            self.handle = None


class Stream:
    """An in-order HIP stream: the command buffer + encoder of ComputeContext."""

    def __init__(self, device: AudioDevice):
        h = C.c_void_p()
        check(lib().mnn_stream_create(device.handle, C.byref(h)))
        self.handle = h
        self.device = device

    def sync(self, timeout_ms: int = 0) -> None:
        """Waits for the stream; MNN_ERR_GPU_TIMEOUT after timeout_ms (> 0)."""
        check(lib().mnn_stream_sync(self.handle, int(timeout_ms)))

    def close(self) -> None:
        if self.handle:
            check(lib().mnn_stream_destroy(self.handle))
            self.handle = None


def _sh(stream: Optional[Stream]):
    return stream.handle if stream is not None else None


def bf16_bits(a) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even, NaN kept quiet."""
    u = _f32(a).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


class Tensor:
    """Device tensor, contiguous row-major, zero-initialised (Tensor.swift:59-141); fp32 or bf16
    (dtype "bf16": 16-bit values, host data rounded to nearest even on upload, widened to fp32
    on download)."""

    def __init__(self, device: AudioDevice, shape: Sequence[int], _handle=None, _owned=True,
                 dtype: str = "f32"):
        self.device = device
        self.dtype = dtype
        if _handle is None:
            h = C.c_void_p()
            shape = [int(s) for s in shape]
            check(lib().mnn_tensor_create(device.handle, {"f32": 0, "bf16": 1}[dtype],
                                          len(shape), dims(shape), C.byref(h)))
            _handle = h
        self.handle = _handle
        self._owned = _owned

    @classmethod
    def from_numpy(cls, device: AudioDevice, arr, stream: Optional[Stream] = None,
                   dtype: str = "f32") -> "Tensor":
        a = _f32(arr)
        t = cls(device, a.shape, dtype=dtype)
        t.copy_from(a, stream)
        return t

    @property
    def shape(self) -> tuple[int, ...]:
        r = C.c_int()
        d = dims([])
        check(lib().mnn_tensor_shape(self.handle, C.byref(r), d))
        return tuple(d[i] for i in range(r.value))

    @property
    def count(self) -> int:
        return int(np.prod(self.shape))

    def reshape(self, shape: Sequence[int]) -> None:
        check(lib().mnn_tensor_reshape(self.handle, len(shape), dims(shape)))

    def copy_from(self, arr, stream: Optional[Stream] = None) -> None:
        """Tensor.copy(from:) — synchronous upload."""
        a = _f32(arr)
        if self.dtype == "bf16":
            a = np.ascontiguousarray(bf16_bits(a))
        check(lib().mnn_tensor_upload(self.handle, a.ctypes.data, a.nbytes, _sh(stream)))

    def to_numpy(self, stream: Optional[Stream] = None) -> np.ndarray:
        """toArray() — synchronous download, shaped like the tensor (fp32)."""
        if self.dtype == "bf16":
            raw = np.empty(self.shape, dtype=np.uint16)
            check(lib().mnn_tensor_download(self.handle, raw.ctypes.data, raw.nbytes,
                                            _sh(stream)))
            return (raw.astype(np.uint32) << 16).view(np.float32)
        out = np.empty(self.shape, dtype=np.float32)
        check(lib().mnn_tensor_download(self.handle, out.ctypes.data, out.nbytes, _sh(stream)))
        return out

    def copy_to(self, dst: "Tensor", stream: Optional[Stream] = None) -> None:
        check(lib().mnn_tensor_copy(dst.handle, self.handle, _sh(stream)))

    @property
    def device_ptr(self) -> int:
        p = C.c_void_p()
        check(lib().mnn_tensor_device_ptr(self.handle, C.byref(p)))
        return p.value or 0

    def close(self) -> None:
        if self.handle and self._owned:
            check(lib().mnn_tensor_destroy(self.handle))
        self.handle = None

    def __del__(self):
        try:
            if getattr(self, "handle", None) and self._owned and lib is not None:
                lib().mnn_tensor_destroy(self.handle)
        except Exception:
            pass


class Layer:
    """The NNLayer protocol (NNLayer.swift:12-16) over a C-ABI layer handle."""

    def __init__(self, device: AudioDevice, handle):
        self.device = device
        self.handle = handle

    def load_weights_named(self, name: str, values) -> None:
        a = _f32(values).ravel()
        check(lib().mnn_layer_load_weights(
            self.handle, name.encode(), a.ctypes.data_as(C.POINTER(C.c_float)), a.size))

    def forward(self, input: Tensor, output: Tensor, stream: Optional[Stream] = None) -> None:
        check(lib().mnn_layer_forward(self.handle, input.handle, output.handle, _sh(stream)))

    def _shape(self, fn) -> tuple[int, ...]:
        r = C.c_int()
        d = dims([])
        check(fn(self.handle, C.byref(r), d))
        return tuple(d[i] for i in range(r.value))

    @property
    def input_shape(self) -> tuple[int, ...]:
        return self._shape(lib().mnn_layer_input_shape)

    @property
    def output_shape(self) -> tuple[int, ...]:
        return self._shape(lib().mnn_layer_output_shape)

    def infer_output_shape(self, shape: Sequence[int]) -> tuple[int, ...]:
        r = C.c_int()
        d = dims([])
        check(lib().mnn_layer_infer_output_shape(self.handle, len(shape), dims(shape), C.byref(r), d))
        return tuple(d[i] for i in range(r.value))

    def __call__(self, input: Tensor, stream: Optional[Stream] = None) -> Tensor:
        """Allocates the output, runs forward, returns the output tensor."""
        out = Tensor(self.device, self.infer_output_shape(input.shape))
        self.forward(input, out, stream)
        return out

    def close(self) -> None:
        if self.handle:
            check(lib().mnn_layer_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            if getattr(self, "handle", None):
                lib().mnn_layer_destroy(self.handle)
        except Exception:
            pass


def _create(fn, *args) -> C.c_void_p:
    h = C.c_void_p()
    check(fn(*args, C.byref(h)))
    return h


class Conv1D(Layer):
    """Conv1D (Conv1D.swift:56-103) with FusedConv1D's activation; weight [out, in/groups, k]."""

    def __init__(self, device, input_channels, output_channels, kernel_size, stride=1, padding=0,
                 dilation=1, groups=1, use_bias=True, input_length=0, padding_mode=None,
                 activation="none", precision="f32", leaky_relu_alpha=None):
        if padding_mode is None:
            padding_mode = "explicit"
        d = Conv1dDesc(input_channels, output_channels, kernel_size, stride, padding, dilation,
                       groups, int(use_bias), int(input_length), PAD[padding_mode], ACT[activation],
                       PRECISION[precision])
        if leaky_relu_alpha is None:
            h = _create(lib().mnn_conv1d_create, device.handle, C.byref(d))
        else:
            h = _create(lib().mnn_fused_conv1d_create, device.handle, C.byref(d),
                        float(leaky_relu_alpha))
        super().__init__(device, h)
        self.use_bias = use_bias

    def load_weights(self, weights, bias=None) -> None:
        self.load_weights_named("weight", weights)
        if bias is not None and self.use_bias:
            self.load_weights_named("bias", bias)

    def forward_with_residual(self, input: Tensor, residual: Optional[Tensor], output: Tensor,
                              stream: Optional[Stream] = None) -> None:
        """FusedConv1D.forwardWithResidual: output = act(conv + bias) + residual."""
        check(lib().mnn_conv1d_forward_residual(self.handle, input.handle,
                                                residual.handle if residual else None,
                                                output.handle, _sh(stream)))


class FusedConv1D(Conv1D):
    """FusedConv1D (Conv1D.swift:742-1028): activation (default relu, as the reference) and
    leakyReluAlpha (default 0.01)."""

    def __init__(self, device, input_channels, output_channels, kernel_size, stride=1, padding=0,
                 dilation=1, groups=1, use_bias=True, activation="relu", leaky_relu_alpha=0.01,
                 input_length=0):
        super().__init__(device, input_channels, output_channels, kernel_size, stride, padding,
                         dilation, groups, use_bias, input_length, "explicit", activation,
                         leaky_relu_alpha=leaky_relu_alpha)


class DynamicConv1D(Conv1D):
    """DynamicConv1D (DynamicConv1D.swift:35-403): padding_mode valid/same/explicit/reflect."""

    def __init__(self, device, input_channels, output_channels, kernel_size, stride=1,
                 padding_mode="valid", padding=0, dilation=1, groups=1, use_bias=True,
                 activation="none", precision="f32"):
        super().__init__(device, input_channels, output_channels, kernel_size, stride, padding,
                         dilation, groups, use_bias, 0, padding_mode, activation, precision)


class GroupNorm(Layer):
    def __init__(self, device, num_groups, num_channels, epsilon=1e-5, affine=True,
                 activation="none"):
        super().__init__(device, _create(lib().mnn_groupnorm_create, device.handle, num_groups,
                                         num_channels, epsilon, int(affine), ACT[activation]))

    def load_parameters(self, weight, bias) -> None:
        self.load_weights_named("weight", weight)
        self.load_weights_named("bias", bias)


class LayerNorm(Layer):
    def __init__(self, device, feature_size, epsilon=1e-5):
        super().__init__(device, _create(lib().mnn_layernorm_create, device.handle, feature_size,
                                         epsilon))

    def load_parameters(self, gamma, beta) -> None:
        self.load_weights_named("gamma", gamma)
        self.load_weights_named("beta", beta)


class GELU(Layer):
    def __init__(self, device, input_shape):
        super().__init__(device, _create(lib().mnn_gelu_create, device.handle, len(input_shape),
                                         dims(input_shape)))


class GLU(Layer):
    def __init__(self, device, out_channels):
        super().__init__(device, _create(lib().mnn_glu_create, device.handle, out_channels))


class Linear(Layer):
    def __init__(self, device, input_features, output_features, use_bias=True, activation="none",
                 precision="f32", leaky_relu_alpha=None):
        if leaky_relu_alpha is None:
            h = _create(lib().mnn_linear_create, device.handle, input_features, output_features,
                        int(use_bias), ACT[activation], PRECISION[precision])
        else:
            h = _create(lib().mnn_fused_linear_create, device.handle, input_features,
                        output_features, int(use_bias), ACT[activation], float(leaky_relu_alpha),
                        PRECISION[precision])
        super().__init__(device, h)
        self.use_bias = use_bias

    def load_weights(self, weights, bias=None) -> None:
        self.load_weights_named("weight", weights)
        if bias is not None and self.use_bias:
            self.load_weights_named("bias", bias)


class FusedLinear(Linear):
    """FusedLinear (Linear.swift:475-672): activation (default relu) and leakyReluAlpha."""

    def __init__(self, device, input_features, output_features, use_bias=True, activation="relu",
                 leaky_relu_alpha=0.01, precision="f32"):
        super().__init__(device, input_features, output_features, use_bias, activation,
                         precision, leaky_relu_alpha=leaky_relu_alpha)


class MultiHeadAttention(Layer):
    def __init__(self, device, embed_dim, num_heads, use_bias=True, precision="f32"):
        super().__init__(device, _create(lib().mnn_mha_create, device.handle, embed_dim,
                                         num_heads, int(use_bias), PRECISION[precision]))
        self.use_bias = use_bias

    def load_weights(self, in_proj_weight, in_proj_bias, out_proj_weight, out_proj_bias) -> None:
        self.load_weights_named("in_proj_weight", in_proj_weight)
        self.load_weights_named("out_proj_weight", out_proj_weight)
        if self.use_bias:
            if in_proj_bias is not None:
                self.load_weights_named("in_proj_bias", in_proj_bias)
            if out_proj_bias is not None:
                self.load_weights_named("out_proj_bias", out_proj_bias)

    def forward_cross(self, query: Tensor, key_value: Tensor, output: Tensor,
                      stream: Optional[Stream] = None) -> None:
        check(lib().mnn_layer_forward_cross(self.handle, query.handle, key_value.handle,
                                            output.handle, None, _sh(stream)))


class CrossAttention(MultiHeadAttention):
    """CrossAttention (Attention.swift:986-1063): Q from one sequence, K/V from another."""


class FeedForward(Layer):
    def __init__(self, device, input_dim, hidden_dim, precision="f32"):
        super().__init__(device, _create(lib().mnn_feedforward_create, device.handle, input_dim,
                                         hidden_dim, PRECISION[precision]))

    def load_weights(self, linear1_weight, linear1_bias, linear2_weight, linear2_bias) -> None:
        self.load_weights_named("linear1.weight", linear1_weight)
        self.load_weights_named("linear1.bias", linear1_bias)
        self.load_weights_named("linear2.weight", linear2_weight)
        self.load_weights_named("linear2.bias", linear2_bias)


class UNetEncoderBlock(Layer):
    """UNetEncoderBlock (UNet.swift:11-174), optionally with the 1x1 C->2C rewrite + GLU."""

    def __init__(self, device, input_channels, output_channels, kernel_size=8, stride=4,
                 num_groups=8, rewrite=False, precision="f32"):
        d = EncoderBlockDesc(input_channels, output_channels, kernel_size, stride, num_groups,
                             int(rewrite), PRECISION[precision])
        super().__init__(device, _create(lib().mnn_encoder_block_create, device.handle, C.byref(d)))

    def load_weights(self, conv_weight, conv_bias, norm_weight, norm_bias, rewrite_weight=None,
                     rewrite_bias=None) -> None:
        self.load_weights_named("conv.weight", conv_weight)
        if conv_bias is not None:
            self.load_weights_named("conv.bias", conv_bias)
        self.load_weights_named("norm.weight", norm_weight)
        self.load_weights_named("norm.bias", norm_bias)
        if rewrite_weight is not None:
            self.load_weights_named("rewrite.weight", rewrite_weight)
        if rewrite_bias is not None:
            self.load_weights_named("rewrite.bias", rewrite_bias)

    def forward_alloc(self, input: Tensor, stream: Optional[Stream] = None):
        """forward(input:encoder:) -> (output, skip); the skip is the output itself."""
        out = self(input, stream)
        return out, out


class ConvTranspose1D(Layer):
    """DynamicConvTranspose1D (DynamicConv1D.swift:411-645); weight [in, out/groups, k]."""

    def __init__(self, device, input_channels, output_channels, kernel_size, stride=1, padding=0,
                 output_padding=0, dilation=1, groups=1, use_bias=True):
        d = ConvTranspose1dDesc(input_channels, output_channels, kernel_size, stride, padding,
                                output_padding, dilation, groups, int(use_bias))
        super().__init__(device, _create(lib().mnn_conv_transpose1d_create, device.handle,
                                         C.byref(d)))
        self.stride, self.padding, self.output_padding = stride, padding, output_padding
        self.kernel_size, self.dilation, self.use_bias = kernel_size, dilation, use_bias

    def output_length(self, input_length: int) -> int:
        """outputLength(for:) (DynamicConv1D.swift:483-487)."""
        return ((input_length - 1) * self.stride - 2 * self.padding
                + self.dilation * (self.kernel_size - 1) + self.output_padding + 1)

    def load_weights(self, weights, bias=None) -> None:
        self.load_weights_named("weight", weights)
        if bias is not None and self.use_bias:
            self.load_weights_named("bias", bias)


DynamicConvTranspose1D = ConvTranspose1D


class UNetDecoderBlock(Layer):
    """UNetDecoderBlock (UNet.swift:184-388): concat(input, skip) -> ConvTranspose1D -> GroupNorm
    -> GELU; forward(input, skip)."""

    def __init__(self, device, input_channels, skip_channels, output_channels, kernel_size=8,
                 stride=4, num_groups=8):
        d = DecoderBlockDesc(input_channels, skip_channels, output_channels, kernel_size, stride,
                             num_groups)
        super().__init__(device, _create(lib().mnn_decoder_block_create, device.handle,
                                         C.byref(d)))

    def load_weights(self, conv_transpose_weight, conv_transpose_bias, norm_weight,
                     norm_bias) -> None:
        self.load_weights_named("conv_tr.weight", conv_transpose_weight)
        if conv_transpose_bias is not None:
            self.load_weights_named("conv_tr.bias", conv_transpose_bias)
        self.load_weights_named("norm.weight", norm_weight)
        self.load_weights_named("norm.bias", norm_bias)

    def forward(self, input: Tensor, skip: Tensor, output: Tensor,  # type: ignore[override]
                stream: Optional[Stream] = None) -> None:
        check(lib().mnn_layer_forward_cross(self.handle, input.handle, skip.handle,
                                            output.handle, None, _sh(stream)))

    def forward_alloc(self, input: Tensor, skip: Tensor,
                      stream: Optional[Stream] = None) -> Tensor:
        out = Tensor(self.device, self.infer_output_shape(input.shape))
        self.forward(input, skip, out, stream)
        return out


def unet_padding(input_length: int, levels: int, kernel_size: int = 8,
                 stride: int = 4) -> tuple[int, int, int]:
    """UNetPaddingCalculator.calculatePadding (UNet.swift:393-430): (left, right, padded length)."""
    lp, rp, ol = C.c_int64(), C.c_int64(), C.c_int64()
    check(lib().mnn_unet_padding(input_length, levels, kernel_size, stride, C.byref(lp),
                                 C.byref(rp), C.byref(ol)))
    return lp.value, rp.value, ol.value


def unet_bottleneck_length(input_length: int, levels: int, stride: int = 4) -> int:
    """UNetPaddingCalculator.bottleneckLength (UNet.swift:432-447)."""
    out = C.c_int64()
    check(lib().mnn_unet_bottleneck_length(input_length, levels, stride, C.byref(out)))
    return out.value


def _pair(v) -> tuple[int, int]:
    return (v, v) if isinstance(v, int) else (int(v[0]), int(v[1]))


class Conv2D(Layer):
    """DynamicConv2D (DynamicConv2D.swift:37-592); weight [out, in/groups, kh, kw]. padding:
    "valid", "same", "explicit" or "reflect" (the last two with `pad` = (h, w))."""

    def __init__(self, device, input_channels, output_channels, kernel_size, stride=1,
                 padding="valid", pad=0, dilation=1, groups=1, use_bias=True):
        (kh, kw), (sh, sw), (ph, pw), (dh, dw) = map(_pair, (kernel_size, stride, pad, dilation))
        d = Conv2dDesc(input_channels, output_channels, kh, kw, sh, sw, PAD[padding], ph, pw, dh,
                       dw, groups, int(use_bias))
        super().__init__(device, _create(lib().mnn_conv2d_create, device.handle, C.byref(d)))
        self.use_bias = use_bias

    def load_weights(self, weights, bias=None) -> None:
        self.load_weights_named("weight", weights)
        if bias is not None and self.use_bias:
            self.load_weights_named("bias", bias)


DynamicConv2D = Conv2D


class ConvTranspose2D(Layer):
    """DynamicConvTranspose2D (DynamicConv2D.swift:598-959); weight [in, out/groups, kh, kw]."""

    def __init__(self, device, input_channels, output_channels, kernel_size, stride=1, padding=0,
                 output_padding=0, dilation=1, groups=1, use_bias=True):
        (kh, kw), (sh, sw), (ph, pw), (oph, opw), (dh, dw) = map(
            _pair, (kernel_size, stride, padding, output_padding, dilation))
        d = ConvTranspose2dDesc(input_channels, output_channels, kh, kw, sh, sw, ph, pw, oph, opw,
                                dh, dw, groups, int(use_bias))
        super().__init__(device, _create(lib().mnn_conv_transpose2d_create, device.handle,
                                         C.byref(d)))
        self.use_bias = use_bias

    def load_weights(self, weights, bias=None) -> None:
        self.load_weights_named("weight", weights)
        if bias is not None and self.use_bias:
            self.load_weights_named("bias", bias)


DynamicConvTranspose2D = ConvTranspose2D


class FreqUNetEncoderBlock2D(Layer):
    """FreqUNetEncoderBlock2D (FreqUNet2D.swift:12-192): Conv2D (reflect padding (k-1)/2, stride)
    -> GroupNorm -> GELU; the output is also the block's skip."""

    def __init__(self, device, input_channels, output_channels, kernel_size=3, stride=2,
                 num_groups=8):
        (kh, kw), (sh, sw) = _pair(kernel_size), _pair(stride)
        d = FreqBlockDesc(input_channels, 0, output_channels, kh, kw, sh, sw, num_groups)
        super().__init__(device, _create(lib().mnn_freq_encoder_block_create, device.handle,
                                         C.byref(d)))

    def load_weights(self, conv_weight, conv_bias, norm_weight, norm_bias) -> None:
        self.load_weights_named("conv.weight", conv_weight)
        if conv_bias is not None:
            self.load_weights_named("conv.bias", conv_bias)
        self.load_weights_named("norm.weight", norm_weight)
        self.load_weights_named("norm.bias", norm_bias)


class FreqUNetDecoderBlock2D(UNetDecoderBlock):
    """FreqUNetDecoderBlock2D (FreqUNet2D.swift:198-428): concat(input, skip) -> ConvTranspose2D
    (padding (k-1)/2, output padding stride-1) -> GroupNorm -> GELU; forward(input, skip)."""

    def __init__(self, device, input_channels, skip_channels, output_channels, kernel_size=3,
                 stride=2, num_groups=8):
        (kh, kw), (sh, sw) = _pair(kernel_size), _pair(stride)
        d = FreqBlockDesc(input_channels, skip_channels, output_channels, kh, kw, sh, sw,
                          num_groups)
        Layer.__init__(self, device, _create(lib().mnn_freq_decoder_block_create, device.handle,
                                             C.byref(d)))


STEM_NAMES = ["drums", "bass", "other", "vocals", "guitar", "piano"]


class Separator:
    """Time-domain HTDemucs separation (HTDemucs.swift:260-392, separate :617-691) and the
    long-audio segment driver. Parameters by name: "time_encoder.{i}.*", "time_decoder.{j}.*"
    (j = 0 deepest), "output_heads.{s}.*"."""

    def __init__(self, device, input_channels=2, num_stems=4,
                 channels=(48, 96, 192, 384, 768), kernel_size=8, stride=4, num_groups=8):
        ch = (C.c_int * 8)(*channels)
        d = SeparatorDesc(input_channels, num_stems, len(channels), ch, kernel_size, stride,
                          num_groups)
        h = C.c_void_p()
        check(lib().mnn_separator_create(device.handle, C.byref(d), C.byref(h)))
        self.handle, self.device = h, device
        self.input_channels, self.num_stems = input_channels, num_stems

    def load(self, name: str, data) -> None:
        a = _f32(data).reshape(-1)
        check(lib().mnn_separator_load(self.handle, name.encode(),
                                       a.ctypes.data_as(C.POINTER(C.c_float)), a.size))

    def load_state(self, params: dict) -> None:
        """params: {"time_encoder.0": {"conv.weight": ..., ...}, ...} or flat names."""
        for k, v in params.items():
            if isinstance(v, dict):
                for kk, vv in v.items():
                    self.load(f"{k}.{kk}", vv)
            else:
                self.load(k, v)

    def load_safetensors(self, st: "SafeTensors", mapper: Optional["WeightNameMapper"] = None
                         ) -> int:
        """HTDemucs.loadWeights(from:): the file's time-domain tensors, names mapped by `mapper`
        (detected from the file when None). Returns how many were loaded."""
        m = mapper if mapper is not None else st.create_weight_mapper()
        n = C.c_int()
        check(lib().mnn_separator_load_safetensors(self.handle, st.handle, NAMING[m.convention],
                                                   C.byref(n)))
        return n.value

    def separate(self, x: Tensor, stream: Optional[Stream] = None) -> Tensor:
        out = Tensor(self.device, (self.num_stems, x.shape[0]))
        check(lib().mnn_separator_separate(self.handle, x.handle, out.handle, _sh(stream)))
        return out

    def separate_long(self, x: Tensor, segment_frames: int, overlap_frames: int,
                      stream: Optional[Stream] = None) -> Tensor:
        out = Tensor(self.device, (self.num_stems, x.shape[0]))
        check(lib().mnn_separator_separate_long(self.handle, x.handle, out.handle,
                                                segment_frames, overlap_frames, _sh(stream)))
        return out

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().mnn_separator_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


WINDOWS = {"none": 0, "hann": 1, "hamming": 2, "blackman": 3}


class STFT:
    """STFT (STFT.swift:20-533) on the GPU: `stft(x)` -> (real, imag) tensors, `istft(real, imag)`
    -> signal. layout "frames" = [B?, frames, bins] (STFTResult), "bins" = [B?, bins, frames];
    onesided keeps bins 0..N/2."""

    def __init__(self, device, fft_size: int, hop_size: Optional[int] = None,
                 window: str = "hann"):
        self.device = device
        self.fft_size = fft_size
        self.hop_size = hop_size if hop_size is not None else fft_size // 4
        h = C.c_void_p()
        check(lib().mnn_stft_create(device.handle, fft_size, self.hop_size, WINDOWS[window],
                                    C.byref(h)))
        self.handle = h

    @property
    def window(self) -> np.ndarray:
        out = np.empty(self.fft_size, np.float32)
        check(lib().mnn_stft_window(self.handle, out.ctypes.data_as(C.POINTER(C.c_float)),
                                    self.fft_size))
        return out

    def frame_count(self, samples: int) -> int:
        out = C.c_int64()
        check(lib().mnn_stft_frame_count(self.handle, samples, C.byref(out)))
        return out.value

    def output_length(self, frames: int) -> int:
        out = C.c_int64()
        check(lib().mnn_stft_output_length(self.handle, frames, C.byref(out)))
        return out.value

    def _spec_shape(self, batch, frames, onesided, layout):
        bins = self.fft_size // 2 + 1 if onesided else self.fft_size
        s = (frames, bins) if layout == "frames" else (bins, frames)
        return s if batch is None else (batch,) + s

    def stft(self, x: Tensor, onesided: bool = True, layout: str = "frames",
             stream: Optional[Stream] = None) -> tuple[Tensor, Tensor]:
        batch = x.shape[0] if len(x.shape) == 2 else None
        shp = self._spec_shape(batch, self.frame_count(x.shape[-1]), onesided, layout)
        re, im = Tensor(self.device, shp), Tensor(self.device, shp)
        check(lib().mnn_stft_forward(self.handle, x.handle, re.handle, im.handle, int(onesided),
                                     0 if layout == "frames" else 1, _sh(stream)))
        return re, im

    def istft(self, real: Tensor, imag: Tensor, onesided: bool = True, layout: str = "frames",
              window_floor: float = 1e-10, stream: Optional[Stream] = None) -> Tensor:
        frames = real.shape[-2] if layout == "frames" else real.shape[-1]
        L = self.output_length(frames)
        out = Tensor(self.device, (real.shape[0], L) if len(real.shape) == 3 else (L,))
        check(lib().mnn_stft_inverse(self.handle, real.handle, imag.handle, int(onesided),
                                     0 if layout == "frames" else 1, window_floor, out.handle,
                                     _sh(stream)))
        return out

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().mnn_stft_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def unet_padding_2d(height: int, width: int, levels: int, stride: int = 2):
    """UNetPaddingCalculator2D.calculatePadding (FreqUNet2D.swift:471-497): (top, bottom, left,
    right, padded height, padded width)."""
    out = (C.c_int64 * 6)()
    check(lib().mnn_unet_padding_2d(height, width, levels, stride, out))
    return tuple(out)


def unet_bottleneck_2d(height: int, width: int, levels: int, stride: int = 2):
    """UNetPaddingCalculator2D.bottleneckDimensions (FreqUNet2D.swift:500-512)."""
    out = (C.c_int64 * 2)()
    check(lib().mnn_unet_bottleneck_2d(height, width, levels, stride, out))
    return tuple(out)


ST_DTYPES = ["F32", "F16", "BF16", "I32", "I64", "I16", "I8", "U8", "BOOL"]


class SafeTensors:
    """SafeTensorsLoader (SafeTensorsLoader.swift:41-660) over the C ABI: tensor names, shapes,
    fp32 reads (F32/F16/BF16/integer/bool converted) and loads into layer parameters."""

    def __init__(self, path):
        h = C.c_void_p()
        check(lib().mnn_safetensors_open(str(path).encode(), C.byref(h)))
        self.handle = h

    @property
    def available_tensors(self) -> list[str]:
        n = C.c_int()
        check(lib().mnn_safetensors_tensor_count(self.handle, C.byref(n)))
        out = []
        for i in range(n.value):
            buf = C.create_string_buffer(4096)
            check(lib().mnn_safetensors_tensor_name(self.handle, i, buf, len(buf)))
            out.append(buf.value.decode())
        return out

    def tensor_info(self, name: str) -> tuple[str, tuple[int, ...], int]:
        """(dtype, shape, element count of its bytes)."""
        dt, rank, cnt = C.c_int(), C.c_int(), C.c_size_t()
        d = dims(())
        check(lib().mnn_safetensors_tensor_info(self.handle, name.encode(), C.byref(dt),
                                                C.byref(rank), d, C.byref(cnt)))
        return ST_DTYPES[dt.value], tuple(d[i] for i in range(rank.value)), cnt.value

    def load_tensor(self, name: str) -> np.ndarray:
        """loadTensor(name:) as fp32, shaped."""
        _, shape, count = self.tensor_info(name)
        out = np.empty(count, np.float32)
        check(lib().mnn_safetensors_read_f32(self.handle, name.encode(),
                                             out.ctypes.data_as(C.POINTER(C.c_float)), count))
        return out.reshape(shape) if int(np.prod(shape, dtype=np.int64)) == count else out

    def metadata(self, key: str) -> str:
        buf = C.create_string_buffer(1 << 16)
        check(lib().mnn_safetensors_metadata(self.handle, key.encode(), buf, len(buf)))
        return buf.value.decode()

    def create_weight_mapper(self) -> WeightNameMapper:
        """createWeightMapper(): the convention detected from this file's tensor names."""
        out = C.c_int()
        check(lib().mnn_safetensors_detect_convention(self.handle, C.byref(out)))
        return WeightNameMapper(_NAMING_BY_CODE[out.value])

    def mapped_name(self, metalaudio_name: str, mapper: WeightNameMapper) -> str:
        """The file's own name for `metalaudio_name` (loadTensorMapped's lookup)."""
        return _name_call(lib().mnn_safetensors_find_mapped, self.handle,
                          NAMING[mapper.convention], metalaudio_name.encode())

    def load_tensor_mapped(self, metalaudio_name: str, mapper: WeightNameMapper) -> np.ndarray:
        return self.load_tensor(self.mapped_name(metalaudio_name, mapper))

    def load_into(self, layer: "Layer", tensor_name: str, param_name: str) -> None:
        check(lib().mnn_layer_load_safetensors(layer.handle, self.handle, tensor_name.encode(),
                                               param_name.encode()))

    def close(self) -> None:
        if self.handle:
            lib().mnn_safetensors_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


NAMING = {"metalaudio": 0, "demucs": 1, "unknown": 2}
_NAMING_BY_CODE = {v: k for k, v in NAMING.items()}


def _name_call(fn, *args) -> str:
    buf = C.create_string_buffer(4096)
    check(fn(*args, buf, len(buf)))
    return buf.value.decode()


class WeightNameMapper:
    """WeightNameMapper (WeightNameMapper.swift:7-422): conventions "metalaudio", "demucs" or
    "unknown"; built from a convention or detected from tensor names."""

    def __init__(self, convention: str | None = None, tensor_names: Iterable[str] | None = None):
        if (convention is None) == (tensor_names is None):
            raise ValueError("give either a convention or tensor names")
        if tensor_names is not None:
            convention = self.detect_convention(tensor_names)
        if convention not in NAMING:
            raise ValueError(f"unknown naming convention {convention!r}")
        self.convention = convention

    @staticmethod
    def detect_convention(names: Iterable[str]) -> str:
        enc = [n.encode() for n in names]
        arr = (C.c_char_p * max(1, len(enc)))(*enc)
        out = C.c_int()
        check(lib().mnn_weight_convention_detect(arr, len(enc), C.byref(out)))
        return _NAMING_BY_CODE[out.value]

    def to_metalaudio(self, name: str) -> str:
        return _name_call(lib().mnn_weight_name_to_metalaudio, NAMING[self.convention],
                          name.encode())

    @staticmethod
    def from_metalaudio(name: str, target: str) -> str:
        return _name_call(lib().mnn_weight_name_from_metalaudio, name.encode(), NAMING[target])

    def map_all_to_metalaudio(self, weights: dict) -> dict:
        return {self.to_metalaudio(k): v for k, v in weights.items()}

    def generate_mapping(self, names: Iterable[str]) -> dict:
        return {n: self.to_metalaudio(n) for n in names}

    @staticmethod
    def is_metalaudio_naming(name: str) -> bool:
        out = C.c_int()
        check(lib().mnn_weight_name_is_metalaudio(name.encode(), C.byref(out)))
        return bool(out.value)

    @staticmethod
    def is_demucs_naming(name: str) -> bool:
        out = C.c_int()
        check(lib().mnn_weight_name_is_demucs(name.encode(), C.byref(out)))
        return bool(out.value)


class BinaryModelFile:
    """BinaryModelLoader's "MTLA" files (Model.swift:401-679): read (CRC-32 checked for v2) and
    load into layer parameters; `save` writes version 2."""

    def __init__(self, path):
        h = C.c_void_p()
        check(lib().mnn_mtla_open(str(path).encode(), C.byref(h)))
        self.handle = h

    @property
    def names(self) -> list[str]:
        n = C.c_int()
        check(lib().mnn_mtla_tensor_count(self.handle, C.byref(n)))
        out = []
        for i in range(n.value):
            buf = C.create_string_buffer(1100)
            check(lib().mnn_mtla_tensor_name(self.handle, i, buf, len(buf)))
            out.append(buf.value.decode())
        return out

    def load_tensor(self, name: str) -> np.ndarray:
        rank, cnt = C.c_int(), C.c_size_t()
        d = dims(())
        check(lib().mnn_mtla_tensor_info(self.handle, name.encode(), C.byref(rank), d,
                                         C.byref(cnt)))
        out = np.empty(cnt.value, np.float32)
        check(lib().mnn_mtla_read_f32(self.handle, name.encode(),
                                      out.ctypes.data_as(C.POINTER(C.c_float)), cnt.value))
        return out.reshape(tuple(d[i] for i in range(rank.value)))

    def load_into(self, layer: "Layer", tensor_name: str, param_name: str) -> None:
        check(lib().mnn_layer_load_mtla(layer.handle, self.handle, tensor_name.encode(),
                                        param_name.encode()))

    @staticmethod
    def save(tensors: dict, path) -> None:
        w = C.c_void_p()
        check(lib().mnn_mtla_writer_create(C.byref(w)))
        try:
            for name, arr in tensors.items():
                a = np.ascontiguousarray(arr, dtype=np.float32)
                d = (C.c_int64 * max(1, a.ndim))(*a.shape)
                check(lib().mnn_mtla_writer_add(w, name.encode(), a.ndim, d,
                                                a.ctypes.data_as(C.POINTER(C.c_float))))
            check(lib().mnn_mtla_writer_save(w, str(path).encode()))
        finally:
            lib().mnn_mtla_writer_destroy(w)

    def close(self) -> None:
        if self.handle:
            lib().mnn_mtla_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class TransformerLayer(Layer):
    """Pre-norm MHSA + FFN layer on one sequence; weights named norm1.*, attn.*, norm2.*,
    linear1.*, linear2.*, gamma_1.scale, gamma_2.scale."""

    def __init__(self, device, embed_dim, num_heads, ffn_dim, layer_scale=0.0, precision="f32"):
        super().__init__(device, _create(lib().mnn_transformer_layer_create, device.handle,
                                         embed_dim, num_heads, ffn_dim, layer_scale,
                                         PRECISION[precision]))

    def load_state(self, state: dict) -> None:
        for k, v in state.items():
            self.load_weights_named(k, v)


class CrossTransformerEncoder(Layer):
    """Cross-domain bottleneck; weights layers.{i}.{time|freq}.{norm1|norm2|norm3|attn|linear1|
    linear2|gamma_1|gamma_2}.*"""

    def __init__(self, device, embed_dim, num_heads, ffn_dim, num_layers, layer_scale=1e-4,
                 precision="f32"):
        super().__init__(device, _create(lib().mnn_cross_transformer_create, device.handle,
                                         embed_dim, num_heads, ffn_dim, num_layers, layer_scale,
                                         PRECISION[precision]))

    def load_state(self, state: dict) -> None:
        for k, v in state.items():
            self.load_weights_named(k, v)

    def forward_cross(self, time: Tensor, freq: Tensor, time_out: Tensor, freq_out: Tensor,
                      stream: Optional[Stream] = None) -> None:
        check(lib().mnn_layer_forward_cross(self.handle, time.handle, freq.handle,
                                            time_out.handle, freq_out.handle, _sh(stream)))


class MetalNNCrossTransformerEncoder(CrossTransformerEncoder):
    """CrossTransformerEncoder with the reference class's own layer structure (Transformer.swift:
    370-667): every layer self-attention, cross-attention both ways and an FFN per branch, six LayerNorms, no LayerScale; weights
    layers.{i}.{norm_time_self|...|self_attn_time|...|ffn_freq}.*"""

    def __init__(self, device, embed_dim, num_heads, ffn_dim, num_layers, precision="f32"):
        Layer.__init__(self, device, _create(lib().mnn_cross_transformer_encoder_create,
                                             device.handle, embed_dim, num_heads, ffn_dim,
                                             num_layers, PRECISION[precision]))


class Sequential:
    """Sequential (Model.swift:65-357)."""

    def __init__(self, device: AudioDevice):
        self.device = device
        self.handle = _create(lib().mnn_sequential_create, device.handle)
        self._layers: list[Layer] = []

    def add(self, layer: Layer) -> None:
        check(lib().mnn_sequential_add(self.handle, layer.handle))
        self._layers.append(layer)

    def add_unchecked(self, layer: Layer) -> None:
        check(lib().mnn_sequential_add_unchecked(self.handle, layer.handle))
        self._layers.append(layer)

    def build(self) -> None:
        check(lib().mnn_sequential_build(self.handle))

    def forward(self, input: Tensor, stream: Optional[Stream] = None) -> Tensor:
        """Returns the model-owned output (overwritten by the next forward)."""
        h = C.c_void_p()
        check(lib().mnn_sequential_forward(self.handle, input.handle, _sh(stream), C.byref(h)))
        return Tensor(self.device, (), _handle=h, _owned=False)

    @property
    def buffer_stats(self) -> tuple[int, int]:
        a, n = C.c_int(), C.c_int()
        check(lib().mnn_sequential_buffer_stats(self.handle, C.byref(a), C.byref(n)))
        return a.value, n.value

    @property
    def layer_count(self) -> int:
        n = C.c_int()
        check(lib().mnn_sequential_layer_count(self.handle, C.byref(n)))
        return n.value

    def layer(self, at: int) -> Optional[Layer]:
        """layer(at:) (Model.swift:354-357): the layer object added at that index, or None."""
        h = C.c_void_p()
        check(lib().mnn_sequential_layer_at(self.handle, at, C.byref(h)))
        if not h.value:
            return None
        for l in self._layers:
            if l.handle and C.cast(l.handle, C.c_void_p).value == h.value:
                return l
        raise RuntimeError("layer handle not known to this binding")

    def forward_async(self, input: Tensor, completion, stream: Optional[Stream] = None) -> int:
        """Sequential.forwardAsync (Model.swift:271-346): completion(status, output_or_None) runs
        once, on a library thread after the GPU work (or here, before returning, when the forward
        cannot be enqueued; the status is then also returned). `output` is borrowed as in
        forward()."""
        def trampoline(_user, status, out):
            try:
                completion(status, Tensor(self.device, (), _handle=C.c_void_p(out), _owned=False)
                           if status == 0 and out else None)
            except Exception:  # a raising Python callback must not unwind into the library
                import traceback
                traceback.print_exc()
        cb = _lib.COMPLETION_FN(trampoline)
        self._callbacks = getattr(self, "_callbacks", [])
        self._callbacks.append(cb)  # kept alive until the model is closed
        return lib().mnn_sequential_forward_async(self.handle, input.handle, _sh(stream), cb,
                                                  None)

    def close(self) -> None:
        if self.handle:
            check(lib().mnn_sequential_destroy(self.handle))
            self.handle = None


def mfma_probe(device: AudioDevice, variant: int, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Raw [lane][register] accumulators of one MFMA instruction (see mnn_debug_mfma_probe)."""
    na = 1 if variant < 2 else 8
    nd = 16 if variant in (0, 2) else 4
    a = _f32(a).reshape(64 * na)
    b = _f32(b).reshape(64 * na)
    d = np.zeros(64 * nd, dtype=np.float32)
    fp = C.POINTER(C.c_float)
    check(lib().mnn_debug_mfma_probe(device.handle, variant, a.ctypes.data_as(fp),
                                     b.ctypes.data_as(fp), d.ctypes.data_as(fp)))
    return d.reshape(64, nd)
