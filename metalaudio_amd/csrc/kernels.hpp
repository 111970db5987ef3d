// Host-side launchers of the HIP kernels (one .hip file per kernel family).
#pragma once

#include "common.hpp"

namespace mnn {
namespace k {

// Activation codes follow mnn_activation (FusedConv1D, Conv1D.swift:960-973).
// ------------------------------------------------------------------ elementwise (k_elementwise.hip)
// GELU over n floats; clamp10 = the +-10 passthrough of Activations.swift:124-137.
void gelu(const LaunchCtx& c, const float* x, float* y, int64_t n, bool clamp10);
// y = act(x) for the other activation codes.
void activation(const LaunchCtx& c, const float* x, float* y, int64_t n, int act);
// GLU: per batch b, y[b][i] = x[b][i] * sigmoid(x[b][i + half]) for i < half (NN.metal:1012-1023).
void glu(const LaunchCtx& c, const float* x, float* y, int64_t batch, int64_t half);
void copy_bytes(const LaunchCtx& c, const void* src, void* dst, int64_t bytes);
// d[0 .. n) = 0, as a kernel on the stream (no memset node when the stream is captured).
void zero_u32(const LaunchCtx& c, unsigned* d, int64_t n);
// Measurement floors: an empty launch; one streaming pass reading read_bytes of src and writing
// write_bytes to dst (16-byte aligned, multiples of 16).
void floor_empty(const LaunchCtx& c);
void floor_stream(const LaunchCtx& c, const void* src, int64_t read_bytes, void* dst,
                  int64_t write_bytes);
// fp32 -> bf16 bits, round to nearest even (NaN kept quiet), and bf16 -> fp32 (exact).
void f32_to_bf16(const LaunchCtx& c, const float* x, uint16_t* y, int64_t n);
void bf16_to_f32(const LaunchCtx& c, const uint16_t* x, float* y, int64_t n);

// ------------------------------------------------------------------ norms (k_norm.hip)
// GroupNorm statistics in three steps. x is [B][C][L]; group g covers channels [g*C/G, (g+1)*C/G).
// Step 1 writes per-chunk partials (count, mean, M2) as 3 floats at partials[(bg*nchunk + j)*3].
int gn_num_chunks(int C, int G, int64_t L);
void gn_stats_partial(const LaunchCtx& c, const float* x, int B, int C, int64_t L, int G,
                      float* partials, int nchunk);
// Step 2 merges the nchunk partials of each (b, g) (Chan's parallel formula, fp64, fixed order)
// and writes per-(b, channel) affine coefficients: coef[(b*C + ch)*2 + {0,1}] = {scale, shift},
// scale = gamma[ch]*rstd, shift = beta[ch] - mean*scale, so y = x*scale + shift.
// gamma/beta may be null (affine = false).
void gn_finalize(const LaunchCtx& c, const float* partials, int B, int C, int G, int nchunk,
                 float eps, const float* gamma, const float* beta, float* coef);
// Step 3: y = act(x*scale + shift), per (b, channel) coefficients.
void gn_apply(const LaunchCtx& c, const float* x, float* y, int B, int C, int64_t L,
              const float* coef, int act);
// Steps 2 + 3 in one launch: every workgroup merges the nparts partials of its (b, g) (fp64, a
// fixed order, the same total in every workgroup) and applies y = act(GroupNorm(x)); partials at
// parts[((b*G + g)*nparts + j)*3] (gn_stats_partial's layout, or a producer's for G = 1).
void gn_apply_parts(const LaunchCtx& c, const float* x, float* y, int B, int C, int64_t L, int G,
                    const float* parts, int nparts, const float* gamma, const float* beta,
                    float eps, int act);
// Fixed device scratch for the allocation-free GroupNorm forward: kGnScratchFloats floats per
// GPU (a file-scope __device__ array of k_norm.hip); gn_scratch returns its address on `device`,
// which must be current. Calls that use it concurrently on one GPU race.
constexpr int64_t kGnScratchFloats = 65536;
float* gn_scratch(int device);
// LayerNorm over rows of F features (two-pass statistics, biased variance, rsqrt).
void layernorm(const LaunchCtx& c, const float* x, float* y, int64_t rows, int F,
               const float* gamma, const float* beta, float eps);
// Two LayerNorms of the same rows (own gamma / beta / eps each) in one pass over x where the
// row kernel applies (F % 64 == 0, F <= 512), else two launches.
void layernorm2(const LaunchCtx& c, const float* x, int64_t rows, int F, float* y,
                const float* gamma, const float* beta, float eps, float* y2,
                const float* gamma2, const float* beta2, float eps2);

// (mean, M2) of each 64 consecutive features of every row, parts[rows][F / 64][2] (F % 64 == 0,
// 16-byte aligned rows); with y, x is copied to y in the same pass. The statistics a GEMM with a
// folded LayerNorm (GemmArgs::ln_parts) reads.
void ln_row_parts(const LaunchCtx& c, const float* x, float* y, int64_t rows, int F, float* parts);
// LayerNorm(gamma, beta) folded into the linear map that follows it: Wf = W * diag(gamma) ([N][K]),
// cvec[n] = sum_k Wf[n][k], bf[n] = b[n] + sum_k W[n][k] * beta[k] (b may be null).
void ln_fold(const LaunchCtx& c, const float* W, const float* b, const float* gamma,
             const float* beta, int N, int K, float* Wf, float* cvec, float* bf);

// ------------------------------------------------------------------ conv (k_conv.hip)
struct ConvParams {
  int B, Cin, Cout, Lin, Lout, K, stride, pad, dilation, groups;
  bool reflect;  // reflect padding (DynamicConv1D.swift:288-324) instead of zeros
  int64_t ldy = 0;  // output row pitch (0 = Lout)
  float alpha = 0.01f;  // leaky ReLU slope of the fused activation
  // FusedConv1D residual (Conv1D.swift:1016-1023): y = act(conv + bias) + res, res [B][Cout][ldr]
  // (ldr 0 = ldy); res may alias y.
  const float* res = nullptr;
  int64_t ldr = 0;
};
// Direct convolution, one thread per output position and a block of output channels.
// act: fused activation. If `partials` is set (groups of GroupNorm = 1), each workgroup also
// writes (count, mean, M2) of its outputs (before activation); *nchunk receives the count of
// partials per batch.
// y may be null (statistics only; the register-window kernel).
void conv1d_direct(const LaunchCtx& c, const ConvParams& p, const float* x, const float* w,
                   const float* bias, float* y, int act, float* partials, int* nchunk);
int conv1d_direct_num_chunks(const ConvParams& p);
// True when the register-window kernel runs (it supports statistics-only and fused finalize).
bool conv1d_direct_fusable(const ConvParams& p);
// Conv1D -> GroupNorm(1) -> activation for register-window convolutions (conv1d_direct_fusable):
// pass 1 writes conv_gn_num_parts(p) statistics partials per batch (3 floats each), pass 2
// recomputes the convolution and writes the normalised, activated output once.
int conv_gn_num_parts(const ConvParams& p);
void conv_gn_stats(const LaunchCtx& c, const ConvParams& p, const float* x, const float* w,
                   const float* bias, float* parts);
void conv_gn_apply(const LaunchCtx& c, const ConvParams& p, const float* x, const float* w,
                   const float* bias, const float* parts, int nparts, const float* gamma,
                   const float* beta, float eps, int act, float* y);
// The same chain in one launch, for grids that fit on the device at once (conv_gn_oneshot_fits).
// xch is an exchange buffer of conv_gn_oneshot_exchange_bytes(), zero before its first launch
// (zero_u32) and left ready for the next by each launch. spin_limit bounds each workgroup's wait
// for the others; a workgroup that runs out computes the statistics itself (same result, slower).
// Launches that share xch must not overlap.
size_t conv_gn_oneshot_exchange_bytes();
bool conv_gn_oneshot_fits(const LaunchCtx& c, const ConvParams& p);
void conv_gn_oneshot(const LaunchCtx& c, const ConvParams& p, const float* x, const float* w,
                     const float* bias, void* xch, int spin_limit, const float* gamma,
                     const float* beta, float eps, int act, float* y);
// GEMM tuning override: MNN_GEMM_TILE=<tile id> forces a tile configuration where it applies.

// ------------------------------------------------------------------ GEMM (k_gemm.hip)
// B operand modes. B_KN4 and B_CONVW are the vectorised / windowed forms the launcher picks
// when the operands allow (16-byte aligned rows; conv with k = 8, stride 4, dilation 1).
// B_CONVREC: B[k][n] = act(coef[k].x * conv(x)[k][n] + coef[k].y), conv being a small direct
// conv (Cin * kernel = 16, e.g. the 2-channel first encoder level, weights rc_w [K][16], bias
// rc_b [K]) recomputed while the operand is loaded, so the conv output never goes to HBM.
enum BLayout { B_NK = 0, B_KN = 1, B_CONV = 2, B_KN4 = 3, B_CONVW = 4, B_CONVREC = 5 };
enum BiasMode { BIAS_NONE = 0, BIAS_N = 1, BIAS_M = 2 };

struct GemmArgs {
  int M = 0, N = 0, K = 0, batch = 1;
  // A [M][K], row-major with row stride lda (always K-contiguous)
  const float* A = nullptr;
  int64_t lda = 0, sA = 0;
  // B: B_NK -> [N][K] rows of stride ldb; B_KN -> [K][N] rows of stride ldb (rows may be
  //    padded: ldb >= N, elements between N and ldb are read but never used);
  //    B_CONV -> implicit im2col of x [Cin][conv_L] (row stride ldb):
  //    B[k][n] = x[k / conv_ks][n*conv_stride - conv_pad + (k % conv_ks)*conv_dil]
  const float* B = nullptr;
  int64_t ldb = 0, sB = 0;
  int blayout = B_NK;
  // B_KN on the LDS-DMA path (opt-in, bkn_lds): rows k < kc1 from B, rows kc1 .. kvalid - 1 from
  // B2 (row k - kc1, batch stride sB2), rows past kvalid repeat the last valid row (A's columns
  // there must be zero)
  bool bkn_lds = false;
  const float* B2 = nullptr;
  int64_t sB2 = 0;
  int kc1 = 0, kvalid = 0;
  int conv_L = 0, conv_ks = 1, conv_stride = 1, conv_pad = 0, conv_dil = 1;
  bool conv_reflect = false;
  // Optional prologue on B (B_KN / B_CONVREC): B[k][n] <- act(B[k][n]*scale_k + shift_k); this
  // applies GroupNorm (+GELU) of the producer while loading. The coefficients come either from
  // pro_coef[b][k][2] (batch stride 2*K) or, with pro_stats, from GroupNorm(1) partials
  // (count, mean, M2) of the producer (pro_nparts per batch) merged by every workgroup:
  // scale_k = pro_gamma[k] * rstd, shift_k = pro_beta[k] - mean * scale_k.
  const float* pro_coef = nullptr;
  const float* pro_stats = nullptr;
  int pro_nparts = 0;
  const float* pro_gamma = nullptr;
  const float* pro_beta = nullptr;
  float pro_eps = 1e-5f;
  int pro_act = 0;
  // C [M][N] row-major (or [M/2][N] with glu)
  float* C = nullptr;
  int64_t ldc = 0, sC = 0;
  const float* bias = nullptr;
  int bias_mode = BIAS_NONE;
  int act = 0;
  float act_alpha = 0.01f;  // leaky ReLU slope (act 2)
  // GLU epilogue: rows are stored in 32-row blocks [a0..a15, b0..b15]; output row
  // 16*blk + r = a * sigmoid(b).
  bool glu = false;
  // Residual: C = R + rscale[n] * (act(acc + bias)); R may alias C.
  const float* R = nullptr;
  int64_t ldr = 0, sR = 0;
  const float* rscale = nullptr;
  // GroupNorm(1) statistics of the output (after bias, before act): per workgroup partials
  // (count, mean, M2) at stats[(b*tiles + tile)*3]; tiles = gemm_num_tiles(...)
  float* stats = nullptr;
  // Transposed-conv scatter epilogue (ct_stride = s > 0, LDS path only): row m = s*oc + r, column
  // n = q; C[oc * ldc + s*q + r - ct_pad] = acc + bias[oc] where that position is in [0, ct_len).
  int ct_stride = 0, ct_pad = 0;
  int64_t ct_len = 0;
  // LayerNorm of A's rows folded into the GEMM (LDS path, fp32, row-ordered epilogue, batch 1):
  // B holds W * diag(gamma), bias holds b + W * beta and ln_c[n] = sum_k B[n][k]; the epilogue
  // forms rstd_m * acc - rstd_m * mean_m * ln_c[n] + bias[n] (then activation / residual), with
  // mean_m and rstd_m = 1 / sqrt(var_m + ln_eps) merged from ln_parts: (mean, M2) of each 64
  // consecutive features of row m, [M][K / 64][2].
  const float* ln_parts = nullptr;
  const float* ln_c = nullptr;
  float ln_eps = 1e-5f;
  // Row statistics of the output for a following folded LayerNorm (same path): (mean, M2) of each
  // 64 consecutive columns of the final row m of C, [M][N / 64][2].
  float* row_parts = nullptr;
  // K split (LDS path only): ksplit > 1 writes the raw partial products of each K part to
  // ws[((b * ksplit + p) * M + m) * N + n] and applies no epilogue (the caller reduces the parts).
  int ksplit = 1;
  float* ws = nullptr;
  // B_CONVREC conv: weights [K][16] and bias [K]
  const float* rc_w = nullptr;
  const float* rc_b = nullptr;
  mnn_precision precision = MNN_PRECISION_F32;
  // A and B hold bf16 values (RNE-rounded by their producer), lda / ldb / sA / sB in elements:
  // the LDS-DMA kernel's bf16 instantiation (precision BF16, B_NK, K % 64 == 0).
  bool ab_bf16 = false;
  const char* name = nullptr;  // kernel-timing name of the launch (default: by kernel family)
};
// Number of output tiles per batch for the tile configuration the launcher will pick.
int gemm_num_tiles(const GemmArgs& a);
// Dispatches to the LDS-DMA kernel (k_gemm_lds.hip) when gemm_nk_lds_supported(a), else to the
// register-staged kernel of k_gemm.hip.
void gemm(const LaunchCtx& c, const GemmArgs& a);
// fp32 B_NK GEMM with LDS-DMA operand staging: K % 32 == 0, 16-byte aligned rows, epilogue bias /
// activation / residual with LayerScale, or GLU over 32-row blocks (M % 32 == 0, bias per row, no
// activation or residual); no statistics or B prologue.
bool gemm_nk_lds_supported(const GemmArgs& a);
void gemm_nk_lds(const LaunchCtx& c, const GemmArgs& a);
// Output tiles per batch of the tile gemm_nk_lds would choose for a (fp32 operands; -1 for bf16):
// the number of statistics partials the transposed-conv epilogue writes per batch.
int64_t gemm_nk_lds_tiles(const GemmArgs& a);

// ------------------------------------------------------------------ 2-D conv (k_conv2d.hip)
// DynamicConv2D (DynamicConv2D.swift:37-592): x [B][Cin][H][W] -> y [B][Cout][Ho][Wo], weights
// [Cout][Cin/groups][KH][KW]; zero padding (ph, pw), or mirrored samples with reflect.
struct Conv2DArgs {
  int B = 0, Cin = 0, Cout = 0, H = 0, W = 0, Ho = 0, Wo = 0;
  int KH = 1, KW = 1, sh = 1, sw = 1, ph = 0, pw = 0, dh = 1, dw = 1, groups = 1;
  bool reflect = false;
  const float* x = nullptr;
  const float* w = nullptr;  // direct form: [Cout][Cin/groups][KH][KW]
  const float* bias = nullptr;
  float* y = nullptr;
  int Kp = 0;            // unfold row length (set by conv2d_gemm)
  float* u = nullptr;    // unfold [B][Ho*Wo][Kp] (set by conv2d_gemm)
  // GroupNorm statistics partials of y (count, mean, M2) for stat_groups groups of output
  // channels, conv2d_gemm_stats_parts(a) per (batch, group) in gn_apply_parts' layout, written by
  // the implicit GEMM's split-K reduce (conv2d_gemm)
  float* stats = nullptr;
  int stat_groups = 1;
};
// Matrix-core form (groups 1): weights packed [Cout][conv2d_padded_k] (zero columns past
// Cin*KH*KW) by conv2d_pack_weights; unfold workspace of conv2d_unfold_floats floats (0 for
// pointwise convs, which read the input directly).
int conv2d_padded_k(int Cin, int KH, int KW);
// Few input channels (1 or 2), 3x3 kernel, dilation 1, groups 1, Cout a multiple of 8: a direct
// register-window kernel (no unfold). With stats, GroupNorm partials for G groups as well,
// conv2d_small_parts(a, G) per (batch, group) in gn_apply_parts' layout (0: not available).
bool conv2d_small_supported(const Conv2DArgs& a);
int conv2d_small_parts(const Conv2DArgs& a, int G);
void conv2d_small(const LaunchCtx& c, const Conv2DArgs& a, float* stats, int G);
bool conv2d_gemm_supported(const Conv2DArgs& a);
bool conv2d_pointwise(const Conv2DArgs& a);
int64_t conv2d_unfold_floats(const Conv2DArgs& a);
// The implicit-GEMM form (3x3, padding 1, dilation 1, stride 1 or 2, Cin % 4 == 0,
// Cout % 96 == 0, the input window of 128 output positions within its LDS budget): conv2d_gemm
// then reads the input in place (no unfold workspace).
bool conv2d_igemm_supported(const Conv2DArgs& a);
// Statistics partials per (batch, group) that conv2d_gemm writes when a.stats is set (the
// implicit GEMM split over K, whose reduce pass writes them); 0 where it writes none.
int conv2d_gemm_stats_parts(const Conv2DArgs& a);
// Workspace of the K split conv2d_gemm chooses for small grids (0: no split).
int64_t conv2d_split_ws_floats(const Conv2DArgs& a);
void conv2d_pack_weights(const float* w, int Cout, int Cin, int KH, int KW, float* out);
void conv2d_gemm(const LaunchCtx& c, const Conv2DArgs& a, const float* wpack, float* unfold,
                 float* split_ws);
void conv2d_direct(const LaunchCtx& c, const Conv2DArgs& a);

// DynamicConvTranspose2D (DynamicConv2D.swift:598-959) over the channel concat [x1; x2] (C2 may
// be 0): y [B][Cout][Ho][Wo], weights [C1 + C2][Cout/groups][KH][KW].
struct ConvT2DArgs {
  int B = 0, C1 = 0, C2 = 0, Cout = 0, H = 0, W = 0, Ho = 0, Wo = 0;
  int KH = 1, KW = 1, sh = 1, sw = 1, ph = 0, pw = 0, dh = 1, dw = 1, groups = 1;
  const float* x1 = nullptr;
  const float* x2 = nullptr;
  const float* w = nullptr;  // direct form
  const float* bias = nullptr;
  float* y = nullptr;
  const float* z = nullptr;  // GEMM form: tap products [B][Cout*KH*KW][H*W] (set by convt2d_gemm)
  // GroupNorm statistics partials of y (count, mean, M2) for stat_groups groups of output
  // channels, convt2d_stats_parts(a) per (batch, group) at stats[((b * G + g) * parts + j) * 3]
  // (gn_apply_parts' layout), written by the few-channel kernel or the GEMM form's gather
  float* stats = nullptr;
  int stat_groups = 1;
};
// Matrix-core form (groups 1): weights packed [Cout*KH*KW][convt2d_padded_cin] by
// convt2d_pack_weights; tap-product workspace of convt2d_z_floats floats and an operand
// workspace of convt2d_unfold_floats floats (the input transposed to [H*W][Cp], both inputs).
int convt2d_padded_cin(int Cin);
bool convt2d_gemm_supported(const ConvT2DArgs& a);
int64_t convt2d_z_floats(const ConvT2DArgs& a);
int64_t convt2d_unfold_floats(const ConvT2DArgs& a);
void convt2d_pack_weights(const float* w, int Cin, int Cout, int KH, int KW, float* out);
void convt2d_gemm(const LaunchCtx& c, const ConvT2DArgs& a, const float* wpack, float* z,
                  float* unfold);
// Statistics partials per (batch, group) that convt2d_small or convt2d_gemm writes when a.stats is
// set (the few-channel kernel, or the GEMM form's fixed-kernel gather: 3x3, stride 2, dilation 1);
// 0 where none are written.
int convt2d_stats_parts(const ConvT2DArgs& a);
void convt2d_direct(const LaunchCtx& c, const ConvT2DArgs& a);
// Few output channels (1, 2, 4), 3x3 kernel, stride 2, padding 1, dilation 1, groups 1: a
// direct kernel reading the input in place (no unfold, no tap products).
bool convt2d_small_supported(const ConvT2DArgs& a);
void convt2d_small(const LaunchCtx& c, const ConvT2DArgs& a);

// ------------------------------------------------------------------ separation (k_separate.hip)
// One segment [start, start + len) of interleaved audio x [n][C]: planar padded network input
// xp [C][Lp] (left pad lp), stems y [S][C][Lp] written back into out [S][n][C] with a linear
// crossfade over the first `fade` frames.
struct SegmentArgs {
  int C = 0, S = 0;
  int64_t n = 0, start = 0, len = 0, Lp = 0, lp = 0, fade = 0;
  const float* x = nullptr;
  float* xp = nullptr;
  const float* y = nullptr;
  float* out = nullptr;
};
void segment_deinterleave_pad(const LaunchCtx& c, const SegmentArgs& a);
void segment_crossfade_store(const LaunchCtx& c, const SegmentArgs& a);

// ------------------------------------------------------------------ STFT (k_stft.hip)
// STFT / iSTFT (STFT.swift:40-533): frames of N samples every hop, window win[N]; twiddles
// tw[k] = e^{-2 pi i k / N}, k < N/2 (float2). Spectra are [batch][frames][bins] (layout 0) or
// [batch][bins][frames] (layout 1), bins = N/2 + 1 (onesided) or N.
constexpr int kStftMaxN = 16384;
// The register-resident FFT of the STFT kernels (M = N / 2 = 2^logm, kStftSkMinLogM <= logm <=
// kStftSkMaxLogM) runs Stockham passes of radix 16 and one last pass of the remaining radix; pass
// p >= 1 (L = 16^p points already combined) multiplies by W_{L R}^{r k}, read from the plan's
// table at (L - 16) + (r - 1) L + k (M - 16 entries in all).
constexpr int kStftSkMinLogM = 6, kStftSkMaxLogM = 12;
constexpr int stft_sk_passes(int logm) { return (logm + 3) / 4; }
constexpr int stft_sk_radix(int logm, int p) {
  return p < stft_sk_passes(logm) - 1 ? 16 : 1 << (logm - 4 * (stft_sk_passes(logm) - 1));
}
struct StftArgs {
  int N = 0, logM = 0, hop = 0, batch = 0, onesided = 1, layout = 0;
  int64_t n = 0;       // forward: samples per signal
  int64_t frames = 0;
  const float* win = nullptr;
  const float2* tw = nullptr;
  const float2* stw = nullptr;  // Stockham pass twiddles (register-resident FFT sizes)
  const float* x = nullptr;   // forward input [batch][n]
  float* re = nullptr;        // forward outputs
  float* im = nullptr;
  const float* cre = nullptr; // inverse inputs
  const float* cim = nullptr;
  float* frames_buf = nullptr;  // inverse workspace [batch][frames][N]
  float* y = nullptr;           // inverse output [batch][(frames - 1) * hop + N]
  float floor = 1e-10f;
};
void stft_forward(const LaunchCtx& c, const StftArgs& a);
void stft_inverse(const LaunchCtx& c, const StftArgs& a);

// ------------------------------------------------------------------ transposed conv (k_convt.hip)
// DynamicConvTranspose1D (DynamicConv1D.swift:411-645) over the channel concat [x1; x2] (x2 may be
// absent: C2 = 0): y[b][oc][o] (row pitch Lout) = bias + sum over (ic, k) with
// o = i*stride - pad + k*dil. Weights w [C1 + C2][Cout/groups][K].
struct ConvTArgs {
  int B = 1, C1 = 0, C2 = 0, Cout = 0, K = 0, stride = 1, pad = 0, dil = 1, groups = 1;
  int64_t L = 0, Lout = 0;
  const float* x1 = nullptr;  // [B][C1][L]
  const float* x2 = nullptr;  // [B][C2][L]
  const float* w = nullptr;
  const float* bias = nullptr;
  float* y = nullptr;  // [B][Cout][Lout]
  // GroupNorm statistics partials of y (count, mean, M2) for stat_groups groups of output
  // channels, convt_stats_parts(a) per (batch, group) at stats[((b * G + g) * parts + j) * 3]
  // (gn_apply_parts' layout)
  float* stats = nullptr;
  int stat_groups = 1;
};
struct ConvTPackArgs {
  const float* x1 = nullptr;
  const float* x2 = nullptr;
  int C1 = 0, C2 = 0, Cp = 0;
  int64_t L = 0, Lq = 0;
  float* u = nullptr;  // [B][Lq][T * Cp]
};
// The matrix-core form: groups 1, dilation 1, K = T * stride with T in {1, 2, 4}.
bool convt_gemm_supported(int Cin, int Cout, int K, int stride, int dil, int groups);
// Statistics partials per (batch, group) that convt_gemm writes when a.stats is set (a.stat_groups
// groups): one per output tile for one group (the scatter epilogue), one per reduce workgroup
// for any group count (the split-K reduce); 0 where it writes none (more than one group without a
// K split, or the few-channel kernel, whose partials would be too many for the apply pass's merge).
int convt_stats_parts(const ConvTArgs& a);
int convt_padded_cin(int Cin);
// Output rows q of the GEMM form: (Lout - 1 + pad) / stride + 1.
int64_t convt_rows(int64_t Lout, int stride, int pad);
// Host packing of the weights for the GEMM form: out [stride * Cout][T * Cp],
// out[stride*oc + r][t*Cp + ic] = w[ic][oc][r + stride*t] (zero for padded channels).
void convt_pack_weights(const float* w, int Cin, int Cout, int K, int stride, float* out);
// Floats of the unfolded-input workspace the GEMM form needs.
int64_t convt_unfold_floats(int B, int Cin, int K, int stride, int pad, int64_t Lout);
// The T = 1 operand pack on its own: u[b][q][c] = [x1; x2][c][q] (zero for C1 + C2 <= c < Cp),
// q < L (= Lq); the transposed operand of the 2-D transposed conv's tap GEMM.
void convt_pack_t1(const LaunchCtx& c, const ConvTPackArgs& p, int B);
void convt_gemm(const LaunchCtx& c, const ConvTArgs& a, const float* wpack, float* unfold,
                float* split_ws);
void convt_direct(const LaunchCtx& c, const ConvTArgs& a);
// Workspace floats convt_gemm needs beside the unfold for the K split it will choose.
int64_t convt_split_ws_floats(int B, int Cin, int Cout, int K, int stride, int pad, int64_t Lout);
// Few output channels (k 8, stride 4, Cout 1, 2 or 4): registers per column, no unfold.
bool convt_small_supported(int Cin, int Cout, int K, int stride, int dil, int groups);
void convt_small(const LaunchCtx& c, const ConvTArgs& a);

// ------------------------------------------------------------------ encoder levels (k_enc.hip)
// Strided conv (kernel 8, stride 4, dilation 1, groups 1, pad < 4) as an LDS-DMA implicit GEMM:
// y[b][co][t] (row pitch ldy) = bias + conv. The weights are [Cout][Cinp * 8] with
// Cinp = enc_conv_padded_cin(Cin) (input channels rounded up to 4, the extra taps zero). Writes
// GroupNorm(1) statistics partials (count, mean, M2) of y: enc_conv_parts per batch, 3 floats
// each. Deep levels split K over workgroups: they need a workspace of enc_conv_ws_floats floats.
struct EncConvArgs {
  int B = 1, Cin = 0, Cout = 0;
  int64_t L = 0, Lout = 0;
  int pad = 0;
  bool reflect = true;
  const float* x = nullptr;  // [B][Cin][L]
  const float* w = nullptr;  // [Cout][enc_conv_padded_cin(Cin) * 8]
  const float* bias = nullptr;
  float* y = nullptr;
  int64_t ldy = 0;
  float* parts = nullptr;
  float* ws = nullptr;
  // GroupNorm(1) + GELU in the split-K finish (enc_conv_gn_fits): when zt is set, the K parts are
  // summed by one launch that exchanges the statistics between its workgroups and writes
  // zt [B][Lout][Cout] = GELU(GroupNorm(y))^T (the rewrite's operand); y and parts are unused.
  // xch: the exchange buffer (enc_exchange_bytes, zero before the first launch; epoch-tagged).
  float* zt = nullptr;
  const float* gamma = nullptr;
  const float* beta = nullptr;
  float eps = 1e-5f;
  void* xch = nullptr;
  int spin_limit = 65536;
};
// Bytes of the exchange buffer of the encoder's one-launch GroupNorm forms (first level and the
// split-K finish); one per layer, zeroed once.
size_t enc_exchange_bytes();
// Whether the GroupNorm split-K finish applies: Cout % 32 == 0, a conv the implicit-GEMM kernel
// takes, and a finish grid that is resident at once on this device.
bool enc_conv_gn_fits(const LaunchCtx& c, int Cin, int Cout, int64_t L, int64_t Lout, int B);
bool enc_conv_supported(int Cin, int Cout, int ks, int stride, int dil, int groups, int pad,
                        int64_t L);
int enc_conv_padded_cin(int Cin);
// Statistics partials per batch the launch writes; K = enc_conv_padded_cin(Cin) * 8.
int enc_conv_parts(int Cout, int64_t Lout, int K, int batch);
// Workspace floats of the split-K partial products (0 without a split); gn: the GroupNorm finish
// (which always splits K).
int64_t enc_conv_ws_floats(int Cout, int64_t Lout, int K, int batch, bool gn = false);
// The K split and output tile the conv launcher picks (for measurement accounting).
void enc_conv_plan_info(int Cin, int Cout, int64_t Lout, int batch, bool gn, int* splits,
                        int* bm, int* bn);
void enc_conv(const LaunchCtx& c, const EncConvArgs& a);
// Rewrite 1x1 conv C -> 2C with GLU: out[b][c][t] = z[c] * sigmoid(z[c + C]),
// z = w * GELU(GroupNorm(y)) + bias, in two launches: GroupNorm + GELU of y written transposed to
// zt [B][Lout][kp] (kp = enc_rewrite_kp(C), columns past C zero), then the LDS GEMM with the GLU
// epilogue. w / bias are regrouped into 32-row blocks [a0..a15 | b0..b15] (GLU partners in one
// block) and w is [2C][kp] with zero columns past C. GroupNorm(1) comes from the producer's
// statistics partials (parts, nparts per batch; merged in fp64 in a fixed order) with gamma /
// beta and eps, or from per-row coefficients coef[b][c] = (scale, shift).
struct EncRewriteArgs {
  int B = 1, C = 0;
  int64_t Lout = 0;
  const float* w = nullptr;     // [2C][kp], regrouped
  const float* bias = nullptr;  // [2C], regrouped
  const float* y = nullptr;     // [B][C][ldy]
  int64_t ldy = 0;
  const float* parts = nullptr;
  int nparts = 0;
  float eps = 1e-5f;
  const float* coef = nullptr;
  const float* gamma = nullptr;
  const float* beta = nullptr;
  float* zt = nullptr;  // workspace [B][Lout][kp]
  int kp = 0;
  float* out = nullptr;  // [B][C][ldo]
  int64_t ldo = 0;
  bool zt_ready = false;  // zt already holds GELU(GroupNorm(y))^T: the GEMM only
};
int enc_rewrite_kp(int C);
void enc_rewrite(const LaunchCtx& c, const EncRewriteArgs& a);
// First-level block in two passes (Cin <= 4, C = 48, kernel 8 / stride 4, pad < 4): a statistics
// pass computes the conv on the matrix cores and writes one GroupNorm(1) partial per workgroup
// (enc_l1_parts per batch, into parts); the second pass recomputes the conv with GroupNorm folded
// into its weights and bias, applies GELU on the accumulators, runs the rewrite 48 -> 96 from
// there and GLU; only out [B][48][ldo] is written. a_rw is the rewrite weight, regrouped into
// 32-row GLU blocks ([96][48]), packed by enc_l1_pack_rewrite into the kernel's operand order
// (3 * 24 * 64 floats); rb the regrouped rewrite bias.
int enc_l1_parts(int64_t Lout);
struct EncL1Args {
  int B = 1, Cin = 0, C = 0, pad = 0;
  int64_t L = 0, Lout = 0, ldo = 0;
  bool reflect = true;
  float eps = 1e-5f;
  const float* x = nullptr;      // [B][Cin][L]
  const float* w1 = nullptr;     // conv weight [C][Cin * 8]
  const float* b1 = nullptr;     // conv bias [C] (may be null)
  const float* gamma = nullptr;  // GroupNorm affine (may be null)
  const float* beta = nullptr;
  float* parts = nullptr;        // workspace: 3 * B * enc_l1_parts(Lout) floats
  const float* a_rw = nullptr;
  const float* rb = nullptr;
  float* out = nullptr;
  // One launch instead of two when the grid is resident at once: the workgroups exchange their
  // GroupNorm partials (xch: enc_exchange_bytes, zero before the first launch) and
  // keep the pre-norm conv in LDS; parts is then unused.
  void* xch = nullptr;
  int spin_limit = 65536;
};
constexpr int kEncL1PackFloats = 3 * 24 * 64;
bool enc_l1_supported(int Cin, int Cout, int ks, int stride, int dil, int groups, int pad,
                      int64_t L);
void enc_l1_pack_rewrite(const float* wperm, float* out);
void enc_l1(const LaunchCtx& c, const EncL1Args& a);

// ------------------------------------------------------------------ attention (k_attention.hip)
struct AttnArgs {
  int B = 1, H = 1, Sq = 0, Sk = 0, hd = 0;
  // element (b, s, h, d) of Q is at q[b*q_bs + s*q_rs + h*hd + d]; same for K, V, O.
  const float* q = nullptr;
  int64_t q_bs = 0, q_rs = 0;
  const float* k = nullptr;
  const float* v = nullptr;
  int64_t kv_bs = 0, kv_rs = 0;
  float* o = nullptr;
  int64_t o_bs = 0, o_rs = 0;
  float scale = 1.f;
  // key split: nsplit ranges of the keys run as separate workgroups and a combine step merges
  // them; part is a workspace of attention_part_floats(a, nsplit) floats
  int nsplit = 1;
  float* part = nullptr;
};
// fp32 throughout (operands, scores, softmax, accumulation).
bool attention_supported(int hd);
// Key ranges that fill the device's workgroup slots best for these shapes (1: no split).
int attention_key_splits(const LaunchCtx& c, const AttnArgs& a);
int64_t attention_part_floats(const AttnArgs& a, int nsplit);
void attention(const LaunchCtx& c, const AttnArgs& a);

// ------------------------------------------------------------------ diagnostics (k_probe.hip)
void mfma_probe(const LaunchCtx& c, int variant, const float* a, const float* b, float* d);

}  // namespace k
}  // namespace mnn
