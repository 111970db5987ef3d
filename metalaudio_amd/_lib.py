"""ctypes binding of include/mnn.h (the C ABI of libmnn.so).

Loads the in-tree library metalaudio_amd/lib/libmnn.so. There is no fallback: if the library
is missing or a call fails, an exception is raised.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libmnn.so"
MAX_RANK = 8

# mnn_status
STATUS = {
    0: "MNN_OK",
    1: "MNN_ERR_INVALID_CONFIGURATION",
    2: "MNN_ERR_BUFFER_SIZE_MISMATCH",
    3: "MNN_ERR_PIPELINE_CREATION_FAILED",
    4: "MNN_ERR_GPU_TIMEOUT",
    5: "MNN_ERR_GPU_EXECUTION",
    6: "MNN_ERR_DEVICE_LOST",
    7: "MNN_ERR_OUT_OF_MEMORY",
    8: "MNN_ERR_SHAPE_MISMATCH",
    9: "MNN_ERR_EMPTY_MODEL",
    10: "MNN_ERR_INPUT_SHAPE_MISMATCH",
    11: "MNN_ERR_NOT_BUILT",
    12: "MNN_ERR_INVALID_ARGUMENT",
    13: "MNN_ERR_FILE_NOT_FOUND",
    14: "MNN_ERR_INVALID_FILE",
    15: "MNN_ERR_TENSOR_NOT_FOUND",
}

ACT = {"none": 0, "relu": 1, "leaky_relu": 2, "gelu": 3, "swish": 4, "sigmoid": 5, "tanh": 6}
PAD = {"valid": 0, "same": 1, "explicit": 2, "reflect": 3}
PRECISION = {"f32": 0, "bf16": 1}


class MNNError(RuntimeError):
    """A non-OK mnn_status; `.code` is the status value, `.name` its enum name."""

    def __init__(self, code: int, message: str):
        self.code = code
        self.name = STATUS.get(code, f"status {code}")
        super().__init__(f"{self.name}: {message}")


class Conv1dDesc(C.Structure):
    _fields_ = [
        ("in_channels", C.c_int), ("out_channels", C.c_int), ("kernel_size", C.c_int),
        ("stride", C.c_int), ("padding", C.c_int), ("dilation", C.c_int), ("groups", C.c_int),
        ("use_bias", C.c_int), ("input_length", C.c_int), ("padding_mode", C.c_int),
        ("activation", C.c_int), ("precision", C.c_int),
    ]


class EncoderBlockDesc(C.Structure):
    _fields_ = [
        ("in_channels", C.c_int), ("out_channels", C.c_int), ("kernel_size", C.c_int),
        ("stride", C.c_int), ("num_groups", C.c_int), ("rewrite", C.c_int),
        ("precision", C.c_int),
    ]


class ConvTranspose1dDesc(C.Structure):
    _fields_ = [
        ("in_channels", C.c_int), ("out_channels", C.c_int), ("kernel_size", C.c_int),
        ("stride", C.c_int), ("padding", C.c_int), ("output_padding", C.c_int),
        ("dilation", C.c_int), ("groups", C.c_int), ("use_bias", C.c_int),
    ]


class DecoderBlockDesc(C.Structure):
    _fields_ = [
        ("in_channels", C.c_int), ("skip_channels", C.c_int), ("out_channels", C.c_int),
        ("kernel_size", C.c_int), ("stride", C.c_int), ("num_groups", C.c_int),
    ]


class Conv2dDesc(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "in_channels", "out_channels", "kernel_h", "kernel_w", "stride_h", "stride_w",
        "padding_mode", "pad_h", "pad_w", "dilation_h", "dilation_w", "groups", "use_bias")]


class ConvTranspose2dDesc(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "in_channels", "out_channels", "kernel_h", "kernel_w", "stride_h", "stride_w", "pad_h",
        "pad_w", "output_pad_h", "output_pad_w", "dilation_h", "dilation_w", "groups",
        "use_bias")]


class FreqBlockDesc(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "in_channels", "skip_channels", "out_channels", "kernel_h", "kernel_w", "stride_h",
        "stride_w", "num_groups")]


class SeparatorDesc(C.Structure):
    _fields_ = [("input_channels", C.c_int), ("num_stems", C.c_int), ("levels", C.c_int),
                ("channels", C.c_int * 8), ("kernel_size", C.c_int), ("stride", C.c_int),
                ("num_groups", C.c_int)]


P = C.c_void_p
PP = C.POINTER(C.c_void_p)
I64P = C.POINTER(C.c_int64)
IP = C.POINTER(C.c_int)
FP = C.POINTER(C.c_float)
# void (*mnn_completion_fn)(void* user, mnn_status status, mnn_tensor output)
COMPLETION_FN = C.CFUNCTYPE(None, C.c_void_p, C.c_int, C.c_void_p)

# name -> (restype, argtypes); every function that returns mnn_status uses C.c_int
SIGNATURES = {
    "mnn_last_error_message": (C.c_char_p, []),
    "mnn_status_string": (C.c_char_p, [C.c_int]),
    "mnn_version": (C.c_char_p, []),
    "mnn_device_create": (C.c_int, [C.c_int, PP]),
    "mnn_device_destroy": (C.c_int, [P]),
    "mnn_device_name": (C.c_int, [P, C.c_char_p, C.c_size_t]),
    "mnn_device_synchronize": (C.c_int, [P]),
    "mnn_device_mark_lost": (C.c_int, [P]),
    "mnn_device_check_available": (C.c_int, [P, C.c_int]),
    "mnn_device_set_kernel_timing": (C.c_int, [P, C.c_int]),
    "mnn_device_kernel_timing": (C.c_int, [P, C.c_char_p, I64P, C.POINTER(C.c_double)]),
    "mnn_device_reset_kernel_timing": (C.c_int, [P]),
    "mnn_stream_create": (C.c_int, [P, PP]),
    "mnn_stream_sync": (C.c_int, [P, C.c_int]),
    "mnn_stream_destroy": (C.c_int, [P]),
    "mnn_tensor_create": (C.c_int, [P, C.c_int, C.c_int, I64P, PP]),
    "mnn_tensor_destroy": (C.c_int, [P]),
    "mnn_tensor_shape": (C.c_int, [P, IP, I64P]),
    "mnn_tensor_reshape": (C.c_int, [P, C.c_int, I64P]),
    "mnn_tensor_upload": (C.c_int, [P, P, C.c_size_t, P]),
    "mnn_tensor_download": (C.c_int, [P, P, C.c_size_t, P]),
    "mnn_tensor_copy": (C.c_int, [P, P, P]),
    "mnn_tensor_device_ptr": (C.c_int, [P, PP]),
    "mnn_conv1d_create": (C.c_int, [P, C.POINTER(Conv1dDesc), PP]),
    "mnn_fused_conv1d_create": (C.c_int, [P, C.POINTER(Conv1dDesc), C.c_float, PP]),
    "mnn_conv1d_forward_residual": (C.c_int, [P, P, P, P, P]),
    "mnn_groupnorm_forward_noalloc": (C.c_int, [P, P, P, P]),
    "mnn_groupnorm_create": (C.c_int, [P, C.c_int, C.c_int, C.c_float, C.c_int, C.c_int, PP]),
    "mnn_layernorm_create": (C.c_int, [P, C.c_int, C.c_float, PP]),
    "mnn_gelu_create": (C.c_int, [P, C.c_int, I64P, PP]),
    "mnn_glu_create": (C.c_int, [P, C.c_int, PP]),
    "mnn_linear_create": (C.c_int, [P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, PP]),
    "mnn_fused_linear_create": (
        C.c_int, [P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int, PP]),
    "mnn_mha_create": (C.c_int, [P, C.c_int, C.c_int, C.c_int, C.c_int, PP]),
    "mnn_feedforward_create": (C.c_int, [P, C.c_int, C.c_int, C.c_int, PP]),
    "mnn_encoder_block_create": (C.c_int, [P, C.POINTER(EncoderBlockDesc), PP]),
    "mnn_conv_transpose1d_create": (C.c_int, [P, C.POINTER(ConvTranspose1dDesc), PP]),
    "mnn_decoder_block_create": (C.c_int, [P, C.POINTER(DecoderBlockDesc), PP]),
    "mnn_unet_padding": (C.c_int, [C.c_int64, C.c_int, C.c_int, C.c_int, I64P, I64P, I64P]),
    "mnn_unet_bottleneck_length": (C.c_int, [C.c_int64, C.c_int, C.c_int, I64P]),
    "mnn_separator_create": (C.c_int, [P, C.POINTER(SeparatorDesc), PP]),
    "mnn_separator_destroy": (C.c_int, [P]),
    "mnn_separator_load": (C.c_int, [P, C.c_char_p, FP, C.c_size_t]),
    "mnn_separator_load_safetensors": (C.c_int, [P, P, C.c_int, IP]),
    "mnn_separator_separate": (C.c_int, [P, P, P, P]),
    "mnn_separator_separate_long": (C.c_int, [P, P, P, C.c_int64, C.c_int64, P]),
    "mnn_stft_create": (C.c_int, [P, C.c_int, C.c_int, C.c_int, PP]),
    "mnn_stft_destroy": (C.c_int, [P]),
    "mnn_stft_window": (C.c_int, [P, FP, C.c_size_t]),
    "mnn_stft_frame_count": (C.c_int, [P, C.c_int64, I64P]),
    "mnn_stft_output_length": (C.c_int, [P, C.c_int64, I64P]),
    "mnn_stft_forward": (C.c_int, [P, P, P, P, C.c_int, C.c_int, P]),
    "mnn_stft_inverse": (C.c_int, [P, P, P, C.c_int, C.c_int, C.c_float, P, P]),
    "mnn_conv2d_create": (C.c_int, [P, C.POINTER(Conv2dDesc), PP]),
    "mnn_conv_transpose2d_create": (C.c_int, [P, C.POINTER(ConvTranspose2dDesc), PP]),
    "mnn_freq_encoder_block_create": (C.c_int, [P, C.POINTER(FreqBlockDesc), PP]),
    "mnn_freq_decoder_block_create": (C.c_int, [P, C.POINTER(FreqBlockDesc), PP]),
    "mnn_unet_padding_2d": (C.c_int, [C.c_int64, C.c_int64, C.c_int, C.c_int, I64P]),
    "mnn_unet_bottleneck_2d": (C.c_int, [C.c_int64, C.c_int64, C.c_int, C.c_int, I64P]),
    "mnn_transformer_layer_create": (C.c_int, [P, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int, PP]),
    "mnn_cross_transformer_create": (
        C.c_int, [P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int, PP]),
    "mnn_cross_transformer_encoder_create": (
        C.c_int, [P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, PP]),
    "mnn_safetensors_open": (C.c_int, [C.c_char_p, PP]),
    "mnn_safetensors_close": (C.c_int, [P]),
    "mnn_safetensors_tensor_count": (C.c_int, [P, IP]),
    "mnn_safetensors_tensor_name": (C.c_int, [P, C.c_int, C.c_char_p, C.c_size_t]),
    "mnn_safetensors_tensor_info": (
        C.c_int, [P, C.c_char_p, IP, IP, I64P, C.POINTER(C.c_size_t)]),
    "mnn_safetensors_read_f32": (C.c_int, [P, C.c_char_p, FP, C.c_size_t]),
    "mnn_safetensors_metadata": (C.c_int, [P, C.c_char_p, C.c_char_p, C.c_size_t]),
    "mnn_layer_load_safetensors": (C.c_int, [P, P, C.c_char_p, C.c_char_p]),
    "mnn_weight_convention_detect": (C.c_int, [C.POINTER(C.c_char_p), C.c_int, IP]),
    "mnn_safetensors_detect_convention": (C.c_int, [P, IP]),
    "mnn_weight_name_to_metalaudio": (C.c_int, [C.c_int, C.c_char_p, C.c_char_p, C.c_size_t]),
    "mnn_weight_name_from_metalaudio": (C.c_int, [C.c_char_p, C.c_int, C.c_char_p, C.c_size_t]),
    "mnn_weight_name_is_metalaudio": (C.c_int, [C.c_char_p, IP]),
    "mnn_weight_name_is_demucs": (C.c_int, [C.c_char_p, IP]),
    "mnn_safetensors_find_mapped": (C.c_int, [P, C.c_int, C.c_char_p, C.c_char_p, C.c_size_t]),
    "mnn_mtla_open": (C.c_int, [C.c_char_p, PP]),
    "mnn_mtla_close": (C.c_int, [P]),
    "mnn_mtla_tensor_count": (C.c_int, [P, IP]),
    "mnn_mtla_tensor_name": (C.c_int, [P, C.c_int, C.c_char_p, C.c_size_t]),
    "mnn_mtla_tensor_info": (C.c_int, [P, C.c_char_p, IP, I64P, C.POINTER(C.c_size_t)]),
    "mnn_mtla_read_f32": (C.c_int, [P, C.c_char_p, FP, C.c_size_t]),
    "mnn_layer_load_mtla": (C.c_int, [P, P, C.c_char_p, C.c_char_p]),
    "mnn_mtla_writer_create": (C.c_int, [PP]),
    "mnn_mtla_writer_add": (C.c_int, [P, C.c_char_p, C.c_int, I64P, FP]),
    "mnn_mtla_writer_save": (C.c_int, [P, C.c_char_p]),
    "mnn_mtla_writer_destroy": (C.c_int, [P]),
    "mnn_layer_destroy": (C.c_int, [P]),
    "mnn_layer_load_weights": (C.c_int, [P, C.c_char_p, FP, C.c_size_t]),
    "mnn_layer_forward": (C.c_int, [P, P, P, P]),
    "mnn_layer_forward_cross": (C.c_int, [P, P, P, P, P, P]),
    "mnn_layer_input_shape": (C.c_int, [P, IP, I64P]),
    "mnn_layer_output_shape": (C.c_int, [P, IP, I64P]),
    "mnn_layer_infer_output_shape": (C.c_int, [P, C.c_int, I64P, IP, I64P]),
    "mnn_sequential_create": (C.c_int, [P, PP]),
    "mnn_sequential_destroy": (C.c_int, [P]),
    "mnn_sequential_add": (C.c_int, [P, P]),
    "mnn_sequential_add_unchecked": (C.c_int, [P, P]),
    "mnn_sequential_build": (C.c_int, [P]),
    "mnn_sequential_forward": (C.c_int, [P, P, P, PP]),
    "mnn_sequential_forward_async": (C.c_int, [P, P, P, COMPLETION_FN, P]),
    "mnn_sequential_buffer_stats": (C.c_int, [P, IP, IP]),
    "mnn_sequential_layer_count": (C.c_int, [P, IP]),
    "mnn_sequential_layer_at": (C.c_int, [P, C.c_int, PP]),
    "mnn_debug_mfma_probe": (C.c_int, [P, C.c_int, FP, FP, FP]),
    "mnn_debug_enc_conv_plan": (C.c_int, [C.c_int, C.c_int, C.c_int64, C.c_int, C.c_int, IP, IP,
                                          IP]),
    "mnn_debug_set_launch_log": (C.c_int, [P, C.c_int]),
    "mnn_debug_launch_log": (C.c_int, [P, C.c_char_p, C.c_size_t, C.POINTER(C.c_size_t)]),
    "mnn_debug_set_grid_spin_limit": (C.c_int, [P, C.c_int, C.POINTER(C.c_int)]),
    "mnn_debug_device_allocations": (C.c_int, [I64P]),
    "mnn_debug_empty_launch": (C.c_int, [P]),
    "mnn_debug_stream_rw": (C.c_int, [P, C.c_int64, P, C.c_int64, P]),
    "mnn_debug_stream_mark": (C.c_int, [P, C.c_int]),
    "mnn_debug_kernel_timing_table": (C.c_int, [P, C.c_char_p, C.c_size_t,
                                                C.POINTER(C.c_size_t)]),
    "mnn_debug_stream_mark_elapsed": (C.c_int, [P, C.c_int, C.c_int, C.POINTER(C.c_float)]),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded libmnn.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m metalaudio_amd.build`"
            )
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != 0:
        msg = lib().mnn_last_error_message()
        raise MNNError(status, msg.decode() if msg else "")


def dims(shape) -> C.Array:
    arr = (C.c_int64 * MAX_RANK)()
    for i, v in enumerate(shape):
        arr[i] = int(v)
    return arr
