/*
 * mnn.h — C ABI of the MI355X-native MetalNN inference layer stack.
 *
 * This is the drop-in boundary for the MetalNN hot path of zkeown/MetalAudio:
 * the reference's `NNLayer` protocol (Sources/MetalNN/NNLayer.swift:12-16), the
 * per-layer constructors and loaders, and `Sequential` (Sources/MetalNN/Model.swift:65-357).
 * A Swift package wraps this header as a C target; Python reaches it via ctypes.
 *
 * Conventions
 *  - Every call returns mnn_status (0 = MNN_OK). On failure the thread-local
 *    message from mnn_last_error_message() says what went wrong.
 *  - Handles are opaque and owned by whoever created them. Destroying a layer
 *    that a Sequential still references is the caller's error.
 *  - Tensors are device-resident (HBM), contiguous, row-major, zero-initialised
 *    on creation (reference Tensor.swift:131-139). Host access is explicit
 *    upload/download.
 *  - Work is stream-ordered: a forward enqueues kernels on the stream and
 *    returns; mnn_stream_sync() waits (reference ComputeContext.executeSync,
 *    ComputeContext.swift:154-211). Nothing reads device memory on the host
 *    during a forward, so there are no encode-time read-before-write hazards.
 *  - A layer allocates its workspace on the first forward for a given input
 *    shape and reuses it afterwards; a forward with a shape already seen
 *    allocates nothing. Layers are not safe for concurrent forwards
 *    (reference DynamicConv1D.swift:29-31); use one layer per thread.
 */
#ifndef MNN_H
#define MNN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. 1-7 mirror MetalAudioError (Sources/MetalAudioKit/Core/AudioDevice.swift:11-77);
 * 8-10 mirror SequentialModelError (Sources/MetalNN/Model.swift:5-20). */
typedef enum mnn_status {
  MNN_OK = 0,
  MNN_ERR_INVALID_CONFIGURATION = 1,   /* invalidConfiguration (also NaN/Inf weights, NNLayer.swift:43-48) */
  MNN_ERR_BUFFER_SIZE_MISMATCH = 2,    /* bufferSizeMismatch */
  MNN_ERR_PIPELINE_CREATION_FAILED = 3,/* pipelineCreationFailed: kernel image missing for this GPU */
  MNN_ERR_GPU_TIMEOUT = 4,             /* gpuTimeout (ComputeContext.swift:188-198) */
  MNN_ERR_GPU_EXECUTION = 5,           /* gpuExecutionError (ComputeContext.swift:199-208) */
  MNN_ERR_DEVICE_LOST = 6,             /* deviceLost (AudioDevice.swift:391-472) */
  MNN_ERR_OUT_OF_MEMORY = 7,           /* bufferAllocationFailed */
  MNN_ERR_SHAPE_MISMATCH = 8,          /* SequentialModelError.shapeMismatch */
  MNN_ERR_EMPTY_MODEL = 9,             /* SequentialModelError.emptyModel */
  MNN_ERR_INPUT_SHAPE_MISMATCH = 10,   /* SequentialModelError.inputShapeMismatch */
  MNN_ERR_NOT_BUILT = 11,              /* reserved, never returned: a Sequential used before build() is
                                          MNN_ERR_INVALID_CONFIGURATION "Model not built. Call build()
                                          first.", as the reference (Model.swift:228-229, :293-298) */
  MNN_ERR_INVALID_ARGUMENT = 12,       /* NULL handle, bad rank, unknown weight name */
  /* SafeTensorsLoader.LoaderError (SafeTensorsLoader.swift:95-128) */
  MNN_ERR_FILE_NOT_FOUND = 13,         /* fileNotFound */
  MNN_ERR_INVALID_FILE = 14,           /* headerTooLarge, invalidHeaderJSON, invalidUTF8Header,
                                          offsetOutOfBounds, dataTruncated */
  MNN_ERR_TENSOR_NOT_FOUND = 15        /* tensorNotFound */
} mnn_status;

typedef enum mnn_dtype { MNN_F32 = 0, MNN_BF16 = 1 } mnn_dtype;

/* Compute precision of the matrix products (GEMM, implicit-GEMM conv, attention).
 * F32: fp32 operands on v_mfma_f32_*_f32. BF16: operands rounded to bf16 (RNE),
 * fp32 accumulation (precedent: HalfLinear, HalfPrecisionLinear.swift:60-212).
 * Norms, softmax and activations always run in fp32. */
typedef enum mnn_precision { MNN_PRECISION_F32 = 0, MNN_PRECISION_BF16 = 1 } mnn_precision;

/* Fused activation codes. 0-4 are FusedConv1D's (Conv1D.swift:960-973); FusedLinear's sigmoid
 * and tanh (Linear.swift:630-639) get codes 5 and 6 here. Leaky ReLU's slope is 0.01 (the
 * reference default, Conv1D.swift:786, Linear.swift:495) unless the layer is created with
 * mnn_fused_conv1d_create / mnn_fused_linear_create. GELU is the tanh approximation everywhere
 * (Activations.swift:124-137). */
typedef enum mnn_activation {
  MNN_ACT_NONE = 0, MNN_ACT_RELU = 1, MNN_ACT_LEAKY_RELU = 2, MNN_ACT_GELU = 3, MNN_ACT_SWISH = 4,
  MNN_ACT_SIGMOID = 5, MNN_ACT_TANH = 6
} mnn_activation;

/* DynamicConv1D.PaddingMode (DynamicConv1D.swift:40-61). */
typedef enum mnn_padding_mode {
  MNN_PAD_VALID = 0, MNN_PAD_SAME = 1, MNN_PAD_EXPLICIT = 2, MNN_PAD_REFLECT = 3
} mnn_padding_mode;

typedef struct mnn_device_s* mnn_device;
typedef struct mnn_stream_s* mnn_stream;
typedef struct mnn_tensor_s* mnn_tensor;
typedef struct mnn_layer_s* mnn_layer;
typedef struct mnn_sequential_s* mnn_sequential;

#define MNN_MAX_RANK 8

/* ---------------------------------------------------------------- errors / version */
const char* mnn_last_error_message(void);
const char* mnn_status_string(mnn_status status);
const char* mnn_version(void);

/* ---------------------------------------------------------------- device
 * Replaces AudioDevice(device:) (AudioDevice.swift:323-348). */
mnn_status mnn_device_create(int ordinal, mnn_device* out);
mnn_status mnn_device_destroy(mnn_device dev);
mnn_status mnn_device_name(mnn_device dev, char* buf, size_t buflen);
mnn_status mnn_device_synchronize(mnn_device dev);
/* AudioDevice.markDeviceLost / checkDeviceAvailability (AudioDevice.swift:391-472):
 * after marking, every forward/upload/download on the device fails with MNN_ERR_DEVICE_LOST. */
mnn_status mnn_device_mark_lost(mnn_device dev);
mnn_status mnn_device_check_available(mnn_device dev, int timeout_ms);
/* Per-kernel GPU timing with HIP events, the analogue of executeSyncWithTiming
 * (ComputeContext.swift:232-297). While enabled, every launch of a library kernel is
 * bracketed by events on its stream; mnn_device_kernel_timing() waits for the device and
 * reports the launches and summed milliseconds of kernels whose name contains `kernel_substr`. */
mnn_status mnn_device_set_kernel_timing(mnn_device dev, int enable);
mnn_status mnn_device_kernel_timing(mnn_device dev, const char* kernel_substr,
                                    int64_t* launches, double* total_ms);
mnn_status mnn_device_reset_kernel_timing(mnn_device dev);

/* ---------------------------------------------------------------- stream
 * A stream plays the role of the command buffer + encoder pair. */
mnn_status mnn_stream_create(mnn_device dev, mnn_stream* out);
/* Wait for all work on the stream; MNN_ERR_GPU_TIMEOUT if it is not done within
 * timeout_ms (<= 0 waits without limit). ComputeContext.executeSync, default 2 s (:137). */
mnn_status mnn_stream_sync(mnn_stream s, int timeout_ms);
mnn_status mnn_stream_destroy(mnn_stream s);

/* ---------------------------------------------------------------- tensor
 * Replaces Tensor (Sources/MetalAudioKit/Buffers/Tensor.swift:12-439). */
mnn_status mnn_tensor_create(mnn_device dev, mnn_dtype dtype, int rank, const int64_t* dims,
                             mnn_tensor* out);
mnn_status mnn_tensor_destroy(mnn_tensor t);
mnn_status mnn_tensor_shape(mnn_tensor t, int* rank, int64_t* dims /* [MNN_MAX_RANK] */);
/* Change the shape in place; element count must be unchanged (Tensor views, Tensor.swift:477-511). */
mnn_status mnn_tensor_reshape(mnn_tensor t, int rank, const int64_t* dims);
/* Tensor.copy(from:) / toArray() (Tensor.swift:272-333): copies are ordered on `s`
 * (NULL = the device's default stream) and complete before the call returns. */
mnn_status mnn_tensor_upload(mnn_tensor t, const void* host, size_t bytes, mnn_stream s);
mnn_status mnn_tensor_download(mnn_tensor t, void* host, size_t bytes, mnn_stream s);
/* Device-to-device copy of equal-sized tensors, enqueued on s. */
mnn_status mnn_tensor_copy(mnn_tensor dst, mnn_tensor src, mnn_stream s);
mnn_status mnn_tensor_device_ptr(mnn_tensor t, void** ptr);

/* ---------------------------------------------------------------- layers
 * Every layer implements the NNLayer protocol (NNLayer.swift:12-16): an input shape,
 * an output shape (0 = dynamic dimension, Model.swift:100-104) and forward(input, output). */

typedef struct mnn_conv1d_desc {
  int in_channels, out_channels, kernel_size, stride;
  int padding;          /* used by MNN_PAD_EXPLICIT and MNN_PAD_REFLECT */
  int dilation, groups;
  int use_bias;
  int input_length;     /* > 0: fixed-length Conv1D (Conv1D.swift:56-103); 0: DynamicConv1D */
  mnn_padding_mode padding_mode;
  mnn_activation activation;   /* FusedConv1D epilogue (Conv1D.swift:742-1028) */
  mnn_precision precision;
} mnn_conv1d_desc;

/* Conv1D / DynamicConv1D / FusedConv1D (Conv1D.swift:11-1028, DynamicConv1D.swift:35-403).
 * Weights: "weight" [out, in/groups, k], "bias" [out]. Input [C, L] or [B, C, L]. */
mnn_status mnn_conv1d_create(mnn_device dev, const mnn_conv1d_desc* desc, mnn_layer* out);
/* FusedConv1D.init(..., activation:, leakyReluAlpha:, ...) (Conv1D.swift:775-800): as
 * mnn_conv1d_create with desc->activation fused and leaky_relu_alpha the negative slope of
 * MNN_ACT_LEAKY_RELU (must be finite). */
mnn_status mnn_fused_conv1d_create(mnn_device dev, const mnn_conv1d_desc* desc,
                                   float leaky_relu_alpha, mnn_layer* out);
/* FusedConv1D.forwardWithResidual(input:residual:output:encoder:) (Conv1D.swift:857-900) on any
 * Conv1D layer: output = act(conv(input) + bias) + residual, the residual added AFTER the
 * activation (Conv1D.swift:1016-1023). residual holds as many elements as the output (its
 * shape); NULL gives the plain forward; it may be the output tensor itself. */
mnn_status mnn_conv1d_forward_residual(mnn_layer layer, mnn_tensor input, mnn_tensor residual,
                                       mnn_tensor output, mnn_stream s);

/* GroupNorm (Normalization.swift:32-725); optional fused activation (used by the U-Net block).
 * Parameters "weight"/"gamma" [C], "bias"/"beta" [C]. Input [C, L] or [B, C, L]. */
mnn_status mnn_groupnorm_create(mnn_device dev, int num_groups, int num_channels, float epsilon,
                                int affine, mnn_activation activation, mnn_layer* out);

/* No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The forward of a layer
 * made by mnn_groupnorm_create, as mnn_layer_forward, that allocates nothing: its statistics
 * partials (3 floats per 4096-element chunk of each (batch, group)) go to a fixed scratch of
 * 65536 floats per GPU, held until the process ends, instead of the layer's workspace. Inputs
 * needing more than 21845 partials (batch * groups * ceil(C / groups * L / 4096)) fail with
 * MNN_ERR_INVALID_CONFIGURATION. All calls on one GPU share its scratch: calls that overlap
 * (other streams, other threads) race; calls ordered on one stream do not. */
mnn_status mnn_groupnorm_forward_noalloc(mnn_layer layer, mnn_tensor input, mnn_tensor output,
                                         mnn_stream s);

/* LayerNorm over the last dimension (Normalization.swift:734-964). "gamma"/"weight", "beta"/"bias". */
mnn_status mnn_layernorm_create(mnn_device dev, int feature_size, float epsilon, mnn_layer* out);

/* GELU, tanh approximation with the +-10 clamp (Activations.swift:89-205). */
mnn_status mnn_gelu_create(mnn_device dev, int rank, const int64_t* input_shape, mnn_layer* out);

/* GLU over the channel dimension: [2C, L] -> [C, L] (or [B, 2C, L] -> [B, C, L]),
 * out = a * sigmoid(b), a = first half, b = second half (Shaders/NN.metal:1012-1023). */
mnn_status mnn_glu_create(mnn_device dev, int out_channels, mnn_layer* out);

/* Linear / FusedLinear / HalfLinear (Linear.swift:27-672, HalfPrecisionLinear.swift:60-212):
 * y = act(x W^T + b). "weight" [out, in], "bias" [out]. Input [in], [N, in] or [B, N, in]. */
mnn_status mnn_linear_create(mnn_device dev, int in_features, int out_features, int use_bias,
                             mnn_activation activation, mnn_precision precision, mnn_layer* out);
/* FusedLinear.init(..., activation:, leakyReluAlpha:, ...) (Linear.swift:475-520): as
 * mnn_linear_create with leaky_relu_alpha the negative slope of MNN_ACT_LEAKY_RELU. */
mnn_status mnn_fused_linear_create(mnn_device dev, int in_features, int out_features,
                                   int use_bias, mnn_activation activation,
                                   float leaky_relu_alpha, mnn_precision precision,
                                   mnn_layer* out);

/* MultiHeadAttention / CrossAttention (Attention.swift:15-1063), PyTorch packing:
 * "in_proj_weight" [3E, E] rows Q;K;V, "in_proj_bias" [3E], "out_proj_weight" [E, E],
 * "out_proj_bias" [E]. Input [S, E] or [B, S, E]. Self-attention through mnn_layer_forward,
 * cross-attention through mnn_layer_forward_cross(query, keyValue, output).
 * `precision` applies to the Q/K/V and output projections (MNN_PRECISION_BF16: bf16 operands,
 * fp32 accumulation); the attention core (Q K^T, softmax, P V) always runs in fp32. */
mnn_status mnn_mha_create(mnn_device dev, int embed_dim, int num_heads, int use_bias,
                          mnn_precision precision, mnn_layer* out);

/* FeedForward Linear -> GELU -> Linear (Transformer.swift:7-364).
 * "linear1.weight" [H, E], "linear1.bias" [H], "linear2.weight" [E, H], "linear2.bias" [E]. */
mnn_status mnn_feedforward_create(mnn_device dev, int input_dim, int hidden_dim,
                                  mnn_precision precision, mnn_layer* out);

typedef struct mnn_encoder_block_desc {
  int in_channels, out_channels, kernel_size, stride, num_groups;
  int rewrite;          /* 1: append 1x1 conv C->2C + GLU (the HTDemucs encoder layer) */
  mnn_precision precision;
} mnn_encoder_block_desc;

/* UNetEncoderBlock (UNet.swift:11-174): DynamicConv1D(reflect (k-1)/2) -> GroupNorm -> GELU
 * [-> 1x1 conv C->2C -> GLU]. Weights "conv.weight", "conv.bias", "norm.weight", "norm.bias",
 * "rewrite.weight" [2C, C, 1], "rewrite.bias" [2C]. Input [C, L] or [B, C, L]. The skip output of
 * the reference is the block output itself (UNet.swift:96-97). With GroupNorm(1) and the rewrite
 * (fp32), a grid the device holds at once normalises in one launch per level: the workgroups
 * exchange their statistics through the block's own exchange buffer, so forwards of one block
 * must not overlap on two streams (as its workspaces are shared). */
mnn_status mnn_encoder_block_create(mnn_device dev, const mnn_encoder_block_desc* desc,
                                    mnn_layer* out);

typedef struct mnn_conv_transpose1d_desc {
  int in_channels, out_channels, kernel_size, stride;
  int padding, output_padding, dilation, groups;
  int use_bias;
} mnn_conv_transpose1d_desc;

/* DynamicConvTranspose1D (DynamicConv1D.swift:411-645). Weights "weight" [in, out/groups, k],
 * "bias" [out]. Input [C, L] or [B, C, L]; output length
 * (L - 1) * stride - 2 * padding + dilation * (k - 1) + output_padding + 1. */
mnn_status mnn_conv_transpose1d_create(mnn_device dev, const mnn_conv_transpose1d_desc* desc,
                                       mnn_layer* out);

typedef struct mnn_decoder_block_desc {
  int in_channels, skip_channels, out_channels, kernel_size, stride, num_groups;
} mnn_decoder_block_desc;

/* UNetDecoderBlock (UNet.swift:184-388): concat(input, skip) -> ConvTranspose1D (padding
 * (k-1)/2, output_padding stride-2+k%2) -> GroupNorm -> GELU. Weights "conv_tr.weight"
 * [in+skip, out, k], "conv_tr.bias" [out], "norm.weight", "norm.bias". Forward through
 * mnn_layer_forward_cross(input, skip, output, NULL); input and skip share B and L. */
mnn_status mnn_decoder_block_create(mnn_device dev, const mnn_decoder_block_desc* desc,
                                    mnn_layer* out);

/* ---------------------------------------------------------------- frequency branch (2-D) */
typedef struct mnn_conv2d_desc {
  int in_channels, out_channels, kernel_h, kernel_w, stride_h, stride_w;
  int padding_mode;     /* mnn_padding_mode */
  int pad_h, pad_w;     /* used by MNN_PAD_EXPLICIT and MNN_PAD_REFLECT */
  int dilation_h, dilation_w, groups;
  int use_bias;
} mnn_conv2d_desc;

/* DynamicConv2D (DynamicConv2D.swift:37-592). Weights "weight" [out, in/groups, kh, kw], "bias"
 * [out]. Input [C, H, W] or [B, C, H, W]; output floor((n + 2p - ((k-1)d + 1)) / s) + 1 per
 * axis, "same" padding total/2 per side (computePadding :212-238). */
mnn_status mnn_conv2d_create(mnn_device dev, const mnn_conv2d_desc* desc, mnn_layer* out);

typedef struct mnn_conv_transpose2d_desc {
  int in_channels, out_channels, kernel_h, kernel_w, stride_h, stride_w;
  int pad_h, pad_w, output_pad_h, output_pad_w, dilation_h, dilation_w, groups;
  int use_bias;
} mnn_conv_transpose2d_desc;

/* DynamicConvTranspose2D (DynamicConv2D.swift:598-959). Weights "weight" [in, out/groups, kh, kw],
 * "bias" [out]; output (n-1)s - 2p + (k-1)d + 1 + output_pad per axis. */
mnn_status mnn_conv_transpose2d_create(mnn_device dev, const mnn_conv_transpose2d_desc* desc,
                                       mnn_layer* out);

typedef struct mnn_freq_block_desc {
  int in_channels, skip_channels, out_channels, kernel_h, kernel_w, stride_h, stride_w;
  int num_groups;
} mnn_freq_block_desc;

/* FreqUNetEncoderBlock2D (FreqUNet2D.swift:12-192): Conv2D with reflect padding (k-1)/2 and the
 * stride -> GroupNorm over [C, H*W] -> GELU. skip_channels must be 0. Weights "conv.weight",
 * "conv.bias", "norm.weight", "norm.bias". The block's output is also its skip. */
mnn_status mnn_freq_encoder_block_create(mnn_device dev, const mnn_freq_block_desc* desc,
                                         mnn_layer* out);
/* FreqUNetDecoderBlock2D (FreqUNet2D.swift:198-428): concat(input, skip) -> ConvTranspose2D
 * (padding (k-1)/2, output padding stride-1) -> GroupNorm -> GELU. Weights "conv_tr.weight" (or
 * "conv_transpose.weight"), "conv_tr.bias", "norm.weight", "norm.bias". Two inputs:
 * mnn_layer_forward_cross(input, skip, out). */
mnn_status mnn_freq_decoder_block_create(mnn_device dev, const mnn_freq_block_desc* desc,
                                         mnn_layer* out);
/* UNetPaddingCalculator2D (FreqUNet2D.swift:461-513): out = {pad_top, pad_bottom, pad_left,
 * pad_right, out_height, out_width}; bottleneck = {height, width}. */
mnn_status mnn_unet_padding_2d(int64_t height, int64_t width, int levels, int stride,
                               int64_t out[6]);
mnn_status mnn_unet_bottleneck_2d(int64_t height, int64_t width, int levels, int stride,
                                  int64_t out[2]);

/* STFT / iSTFT (STFT.swift:20-533 over FFT.swift): frames of fft_size samples every hop_size
 * samples (no centring), window applied, full DFT without scaling; spectra [B?, frames, bins]
 * (layout 0, STFTResult's order) or [B?, bins, frames] (layout 1, the frequency branch's
 * spectrogram), bins = fft_size/2 + 1 (onesided) or fft_size. The inverse takes the real part of
 * each frame's inverse DFT (1/N), windows it, overlap-adds and divides by the overlap-added
 * squared window floored at window_floor (STFT.swift:482-531; the reference's default is 1e-10).
 * fft_size: power of 2 in [4, 16384]. */
typedef enum {
  MNN_WINDOW_NONE = 0,
  MNN_WINDOW_HANN = 1,
  MNN_WINDOW_HAMMING = 2,
  MNN_WINDOW_BLACKMAN = 3
} mnn_window;
typedef struct mnn_stft_s* mnn_stft;
mnn_status mnn_stft_create(mnn_device dev, int fft_size, int hop_size, int window, mnn_stft* out);
mnn_status mnn_stft_destroy(mnn_stft plan);
/* WindowType.coefficient(at:length:) for all fft_size indices, into a host array */
mnn_status mnn_stft_window(mnn_stft plan, float* out, size_t count);
mnn_status mnn_stft_frame_count(mnn_stft plan, int64_t samples, int64_t* frames);
mnn_status mnn_stft_output_length(mnn_stft plan, int64_t frames, int64_t* samples);
/* input [n] or [B, n] (f32 tensors on the plan's device) */
mnn_status mnn_stft_forward(mnn_stft plan, mnn_tensor input, mnn_tensor real, mnn_tensor imag,
                            int onesided, int layout, mnn_stream stream);
/* output [L] or [B, L], L = (frames - 1) * hop + fft_size */
mnn_status mnn_stft_inverse(mnn_stft plan, mnn_tensor real, mnn_tensor imag, int onesided,
                            int layout, float window_floor, mnn_tensor output, mnn_stream stream);

/* ---------------------------------------------------------------- separation driver */
/* Time-domain HTDemucs (HTDemucs.swift: time U-Net :260-293 + :521-548, one 1x1 Conv1D output
 * head per stem :333-350, forward :376-392, separate :617-691): interleaved input -> UNet zero
 * padding -> encoders -> decoders with skips -> heads -> crop -> interleaved stems. */
typedef struct mnn_separator_desc {
  int input_channels;   /* 2 (stereo) */
  int num_stems;        /* 4: drums, bass, other, vocals */
  int levels;           /* <= 8 */
  int channels[8];      /* encoder channels per level, e.g. 48, 96, 192, 384, 768 */
  int kernel_size, stride, num_groups;   /* 8, 4, 8 */
} mnn_separator_desc;
typedef struct mnn_separator_s* mnn_separator;
mnn_status mnn_separator_create(mnn_device dev, const mnn_separator_desc* desc,
                                mnn_separator* out);
mnn_status mnn_separator_destroy(mnn_separator sep);
/* "time_encoder.{i}.{conv,norm}.{weight,bias}", "time_decoder.{j}.{conv_transpose|conv_tr,norm}.
 * {weight,bias}" (j = 0 is the deepest level, the order of HTDemucs.loadWeights), and
 * "time_output_heads.{s}.{weight,bias}" (HTDemucs.swift:1021; "output_heads.{s}" also accepted). */
mnn_status mnn_separator_load(mnn_separator sep, const char* name, const float* data, size_t n);
/* HTDemucs.separate(input:mode: .timeOnly) on device tensors: input [n * C] interleaved, output
 * [num_stems, n * C] interleaved stems. */
mnn_status mnn_separator_separate(mnn_separator sep, mnn_tensor input, mnn_tensor output,
                                  mnn_stream stream);
/* Long audio (HTDEMUCS_GUIDE.md:170-191): segments of segment_frames frames starting every
 * segment_frames - overlap_frames frames, each separated as above and written into output with a
 * linear crossfade, weight (i + 1) / (F + 1) for the new segment, over the F frames it shares with
 * the previous one. The guide's crossfadeAppend helper is not defined by the reference; this is
 * the definition used here. segment_frames <= 0 or >= n: one pass. */
mnn_status mnn_separator_separate_long(mnn_separator sep, mnn_tensor input, mnn_tensor output,
                                       int64_t segment_frames, int64_t overlap_frames,
                                       mnn_stream stream);

/* UNetPaddingCalculator (UNet.swift:393-448): left/right zero padding that makes the length a
 * multiple of stride^levels (remainder split evenly, the odd sample on the right), and the length
 * after `levels` downsamplings by `stride`. */
mnn_status mnn_unet_padding(int64_t input_length, int levels, int kernel_size, int stride,
                            int64_t* left_pad, int64_t* right_pad, int64_t* output_length);
mnn_status mnn_unet_bottleneck_length(int64_t input_length, int levels, int stride,
                                      int64_t* length);

/* ---------------------------------------------------------------- weight files
 * SafeTensorsLoader (SafeTensorsLoader.swift:41-660): 8-byte little-endian header length, JSON
 * header, raw data. Entries with a malformed description or an unknown dtype are skipped (as the
 * reference). Reads convert to fp32 (F32, F16, BF16, I32, I64, I16, I8, U8, BOOL) and reject
 * NaN / Inf with MNN_ERR_INVALID_CONFIGURATION. Host-only; one handle is not safe for concurrent
 * reads. */
typedef struct mnn_safetensors_s* mnn_safetensors;
typedef enum mnn_st_dtype {
  MNN_ST_F32 = 0, MNN_ST_F16 = 1, MNN_ST_BF16 = 2, MNN_ST_I32 = 3, MNN_ST_I64 = 4,
  MNN_ST_I16 = 5, MNN_ST_I8 = 6, MNN_ST_U8 = 7, MNN_ST_BOOL = 8
} mnn_st_dtype;
mnn_status mnn_safetensors_open(const char* path, mnn_safetensors* out);
mnn_status mnn_safetensors_close(mnn_safetensors st);
/* availableTensors: the names in sorted order. */
mnn_status mnn_safetensors_tensor_count(mnn_safetensors st, int* count);
mnn_status mnn_safetensors_tensor_name(mnn_safetensors st, int index, char* buf, size_t cap);
/* tensorInfo(name:): dtype, shape (rank <= MNN_MAX_RANK) and the element count of its bytes. */
mnn_status mnn_safetensors_tensor_info(mnn_safetensors st, const char* name, mnn_st_dtype* dtype,
                                       int* rank, int64_t* dims, size_t* count);
/* loadTensor(name:) into `out` (count must equal the tensor's element count). */
mnn_status mnn_safetensors_read_f32(mnn_safetensors st, const char* name, float* out,
                                    size_t count);
/* __metadata__[key] (MNN_ERR_TENSOR_NOT_FOUND when absent). */
mnn_status mnn_safetensors_metadata(mnn_safetensors st, const char* key, char* buf, size_t cap);
/* loadTensor(name:into:) for a layer parameter: reads `tensor_name` and loads it as the layer's
 * parameter `param_name` (mnn_layer_load_weights semantics). */
mnn_status mnn_layer_load_safetensors(mnn_layer layer, mnn_safetensors st,
                                      const char* tensor_name, const char* param_name);

/* Weight-name conventions (WeightNameMapper.swift:7-422): MetalAudio names
 * ("time_encoder.0.conv.weight") and Demucs names ("tencoder.0.conv.weight"). Strings out are
 * NUL-terminated into buf; MNN_ERR_BUFFER_SIZE_MISMATCH when cap is too small. */
typedef enum {
  MNN_NAMES_METALAUDIO = 0,
  MNN_NAMES_DEMUCS = 1,
  MNN_NAMES_UNKNOWN = 2
} mnn_weight_convention;
/* WeightNameMapper.detectConvention(from:) */
mnn_status mnn_weight_convention_detect(const char* const* names, int count, int* convention);
/* SafeTensorsLoader.createWeightMapper(): detection over the file's tensor names */
mnn_status mnn_safetensors_detect_convention(mnn_safetensors st, int* convention);
/* toMetalAudio(name:) for a mapper of `convention` */
mnn_status mnn_weight_name_to_metalaudio(int convention, const char* name, char* buf, size_t cap);
/* fromMetalAudio(name:to:) */
mnn_status mnn_weight_name_from_metalaudio(const char* name, int target, char* buf, size_t cap);
/* isMetalAudioNaming / isDemucsNaming: *out = 0 or 1 */
mnn_status mnn_weight_name_is_metalaudio(const char* name, int* out);
mnn_status mnn_weight_name_is_demucs(const char* name, int* out);
/* loadTensorMapped(metalAudioName:mapper:)'s lookup: the file's own name for the tensor, to pass to
 * mnn_safetensors_read_f32 / mnn_layer_load_safetensors; MNN_ERR_TENSOR_NOT_FOUND if none. */
mnn_status mnn_safetensors_find_mapped(mnn_safetensors st, int convention,
                                       const char* metalaudio_name, char* buf, size_t cap);

/* Separator weights from a SafeTensors file (HTDemucs.loadWeights(from:convention:)) for the
 * time-domain model (mnn_separator, declared with the separation driver): every tensor whose
 * name, mapped from `convention` (mnn_weight_convention) to MetalAudio names, starts with
 * time_encoder. / time_decoder. / time_output_heads. (or output_heads.) is loaded; *loaded = their
 * count. As the reference (HTDemucs.swift:892-937), every encoder conv weight and norm weight /
 * bias and every decoder transposed-conv weight and norm weight / bias must be in the file:
 * otherwise MNN_ERR_TENSOR_NOT_FOUND names the first one missing and nothing is loaded. Conv
 * biases and output heads are optional. */
mnn_status mnn_separator_load_safetensors(mnn_separator sep, mnn_safetensors st, int convention,
                                          int* loaded);

/* "MTLA" binary model files (BinaryModelLoader, Model.swift:401-679): reader (v2 with CRC-32
 * check, legacy v1) and writer (v2, tensors in name order). fp32 tensors, host-only. */
typedef struct mnn_mtla_s* mnn_mtla;
typedef struct mnn_mtla_writer_s* mnn_mtla_writer;
mnn_status mnn_mtla_open(const char* path, mnn_mtla* out);
mnn_status mnn_mtla_close(mnn_mtla m);
mnn_status mnn_mtla_tensor_count(mnn_mtla m, int* count);
mnn_status mnn_mtla_tensor_name(mnn_mtla m, int index, char* buf, size_t cap);
mnn_status mnn_mtla_tensor_info(mnn_mtla m, const char* name, int* rank, int64_t* dims,
                                size_t* count);
mnn_status mnn_mtla_read_f32(mnn_mtla m, const char* name, float* out, size_t count);
mnn_status mnn_layer_load_mtla(mnn_layer layer, mnn_mtla m, const char* tensor_name,
                               const char* param_name);
mnn_status mnn_mtla_writer_create(mnn_mtla_writer* out);
mnn_status mnn_mtla_writer_add(mnn_mtla_writer w, const char* name, int rank, const int64_t* dims,
                               const float* data);
mnn_status mnn_mtla_writer_save(mnn_mtla_writer w, const char* path);
mnn_status mnn_mtla_writer_destroy(mnn_mtla_writer w);

/* Pre-norm transformer layer on one sequence (TransformerLayer sub-blocks 1 and 5,
 * Transformer.swift:467-495): y = x + ls1*MHA(LN1 x); z = y + ls2*FFN(LN2 y).
 * layer_scale <= 0 disables LayerScale. Weights "norm1.*", "self_attn.*", "norm2.*",
 * "linear1.*", "linear2.*", "gamma_1.scale", "gamma_2.scale". Input [S, E] or [B, S, E]. */
mnn_status mnn_transformer_layer_create(mnn_device dev, int embed_dim, int num_heads, int ffn_dim,
                                        float layer_scale, mnn_precision precision,
                                        mnn_layer* out);

/* Cross-domain transformer bottleneck (CrossTransformerEncoder, Transformer.swift:567-700, with
 * the HTDemucs layer structure): num_layers layers, even layers self-attention per branch, odd
 * layers cross-attention (time attends to freq and freq to time, both on pre-update states).
 * forward through mnn_layer_forward_cross(time, freq, time_out, freq_out). Weights
 * "layers.{i}.{time|freq}.{norm1|norm2|norm3|attn|linear1|linear2|gamma_1|gamma_2}.*". */
mnn_status mnn_cross_transformer_create(mnn_device dev, int embed_dim, int num_heads, int ffn_dim,
                                        int num_layers, float layer_scale,
                                        mnn_precision precision, mnn_layer* out);

/* CrossTransformerEncoder(device:embedDim:numHeads:ffnDim:numLayers:) with the reference class's
 * own layer structure (TransformerLayer, Transformer.swift:370-560; layer loop :626-667). Each
 * layer, one residual per sub-block (:467-495): T += SA_t(LN_ts T); F += SA_f(LN_fs F); tn = LN_tc T, fn = LN_fc F; T += CA_t(tn, fn); F += CA_f(fn, tn);
 * T += FFN_t(LN_tf T); F += FFN_f(LN_ff F). No LayerScale. forward through
 * mnn_layer_forward_cross(time, freq, time_out, freq_out); [S, E] or [B, S, E] per branch.
 * Weights as TransformerLayer.loadWeights (:529-557): "layers.{i}.{norm_time_self,
 * norm_freq_self, norm_time_cross, norm_freq_cross, norm_time_ffn, norm_freq_ffn}.{weight,bias}",
 * "layers.{i}.{self_attn_time, self_attn_freq, cross_attn_time, cross_attn_freq}.{in_proj_weight,
 * in_proj_bias, out_proj.weight, out_proj.bias}", "layers.{i}.{ffn_time, ffn_freq}.{linear1,
 * linear2}.{weight,bias}". mnn_cross_transformer_create is the HTDemucs-structured bottleneck of
 * the benchmark configuration instead. */
mnn_status mnn_cross_transformer_encoder_create(mnn_device dev, int embed_dim, int num_heads,
                                                int ffn_dim, int num_layers,
                                                mnn_precision precision, mnn_layer* out);

mnn_status mnn_layer_destroy(mnn_layer layer);
/* loadWeights / loadParameters: copies `count` floats into the named parameter.
 * NaN/Inf are rejected with MNN_ERR_INVALID_CONFIGURATION (validateWeights, NNLayer.swift:27-59);
 * a wrong count gives MNN_ERR_BUFFER_SIZE_MISMATCH. */
mnn_status mnn_layer_load_weights(mnn_layer layer, const char* name, const float* data,
                                  size_t count);
mnn_status mnn_layer_forward(mnn_layer layer, mnn_tensor input, mnn_tensor output, mnn_stream s);
/* Two-input forward: MHA cross-attention (query=a, keyValue=b, output=out_a, out_b unused);
 * cross transformer (time=a, freq=b, time_out=out_a, freq_out=out_b; outputs may alias inputs). */
mnn_status mnn_layer_forward_cross(mnn_layer layer, mnn_tensor a, mnn_tensor b, mnn_tensor out_a,
                                   mnn_tensor out_b, mnn_stream s);
/* Declared shapes (0 = dynamic). */
mnn_status mnn_layer_input_shape(mnn_layer layer, int* rank, int64_t* dims);
mnn_status mnn_layer_output_shape(mnn_layer layer, int* rank, int64_t* dims);
/* Concrete output shape for a concrete input shape. */
mnn_status mnn_layer_infer_output_shape(mnn_layer layer, int in_rank, const int64_t* in_dims,
                                        int* out_rank, int64_t* out_dims);

/* ---------------------------------------------------------------- sequential
 * Sequential (Model.swift:65-357). The model references layers; it does not own them.
 * A Conv1D without activation followed by GroupNorm(1 group) [and GELU] runs as one fused group:
 * for a small contraction whose grid the device holds at once, one launch in which the
 * workgroups exchange their statistics partials through the GroupNorm layer's exchange buffer
 * (so a GroupNorm layer's forwards must not overlap on two streams); otherwise the convolution
 * with statistics from its epilogue (or a statistics pass), then one apply pass. The results are
 * those of the layers run one by one. */
mnn_status mnn_sequential_create(mnn_device dev, mnn_sequential* out);
mnn_status mnn_sequential_destroy(mnn_sequential seq);
mnn_status mnn_sequential_add(mnn_sequential seq, mnn_layer layer);          /* shape-checked */
mnn_status mnn_sequential_add_unchecked(mnn_sequential seq, mnn_layer layer);
/* Ping-pong buffer plan: a layer reuses a same-shape buffer last used >= 2 layers earlier
 * (Model.swift:135-201). Dynamic shapes are resolved on the first forward per input shape. */
mnn_status mnn_sequential_build(mnn_sequential seq);
/* Runs all layers in stream order. *output is borrowed: it belongs to the model and is
 * overwritten by the next forward (Model.swift:263). */
mnn_status mnn_sequential_forward(mnn_sequential seq, mnn_tensor input, mnn_stream s,
                                  mnn_tensor* output);
/* Sequential.forwardAsync(_:completion:) (Model.swift:271-346): enqueues the forward on s and
 * returns. completion(user, status, output) runs exactly once: on a library thread after the GPU
 * work has finished (MNN_OK and the borrowed output, or MNN_ERR_GPU_EXECUTION and NULL), or,
 * when the forward cannot be enqueued, on the calling thread before this returns the same status:
 * MNN_ERR_EMPTY_MODEL, MNN_ERR_INVALID_CONFIGURATION (not built, or another forwardAsync of this
 * model still in flight) or MNN_ERR_INPUT_SHAPE_MISMATCH, as Model.swift:285-320 reports them. As the reference, one forwardAsync per model at a time; the
 * in-flight mark is cleared before the completion runs, so the completion may start the next
 * one. mnn_sequential_destroy waits for the model's completions to return; called from the
 * model's own completion, it waits only for the model's other completions. */
typedef void (*mnn_completion_fn)(void* user, mnn_status status, mnn_tensor output);
mnn_status mnn_sequential_forward_async(mnn_sequential seq, mnn_tensor input, mnn_stream s,
                                        mnn_completion_fn completion, void* user);
mnn_status mnn_sequential_buffer_stats(mnn_sequential seq, int* allocated, int* layers);
mnn_status mnn_sequential_layer_count(mnn_sequential seq, int* count);
/* layer(at:) (Model.swift:354-357): the index-th layer added, or *layer = NULL (status MNN_OK)
 * when index is out of range, as the reference returns nil. The handle is the one passed to
 * mnn_sequential_add. */
mnn_status mnn_sequential_layer_at(mnn_sequential seq, int index, mnn_layer* layer);

#ifdef __cplusplus
}
#endif
#endif /* MNN_H */
