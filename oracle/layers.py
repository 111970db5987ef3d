"""numpy restatement of the MetalNN layer arithmetic (reference: zkeown/MetalAudio).

TEST INFRASTRUCTURE ONLY — see oracle/__init__.py.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "round_bf16", "reflect_pad", "conv1d", "group_norm", "layer_norm", "gelu_tanh", "gelu_layer",
    "stable_sigmoid", "glu", "activation", "fused_conv1d", "linear", "mha", "feed_forward",
    "encoder_block",
    "time_encoder", "conv_transpose1d", "conv_transpose1d_gather", "decoder_block", "unet_padding",
    "unet_bottleneck_length", "time_unet", "transformer_layer", "cross_transformer",
    "cross_transformer_metalnn",
    "reflect_index", "conv2d", "conv2d_output_size", "conv_transpose2d", "freq_encoder_block",
    "freq_decoder_block", "unet_padding_2d",
]

SQRT_2_OVER_PI = 0.7978845608  # literal used by every reference GELU kernel


def _as(x, dtype):
    return np.asarray(x, dtype=dtype)


def round_bf16(x):
    """fp32 -> bf16 -> fp32 with round-to-nearest-even (the operand rounding of the bf16-input /
    fp32-accumulate variant; HalfLinear's fp16 contract, HalfPrecisionLinear.swift:60-212)."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    nan = np.isnan(a)
    if nan.any():
        out = np.where(nan, np.float32(np.nan), out)
    return out.reshape(a.shape)


def reflect_pad(x, pad: int):
    """Reflect padding along the last axis: left x[p..1], right x[L-2..L-1-p].
    Follows DynamicConv1D.applyReflectPadding (DynamicConv1D.swift:288-324)."""
    if pad == 0:
        return x
    L = x.shape[-1]
    if pad >= L:
        raise ValueError("reflect padding needs input length > padding")
    left = x[..., pad:0:-1]                 # reflectIdx = padding - i
    right = x[..., L - 2:L - 2 - pad:-1]    # reflectIdx = inputLength - 2 - i
    return np.concatenate([left, x, right], axis=-1)


def conv1d(x, w, b=None, stride=1, padding=0, dilation=1, groups=1, mode="zeros",
           dtype=np.float64):
    """y[b][co][t] = bias[co] + sum_ci sum_k x[b][ci][t*s - p + k*d] * W[co][ci][k].

    Follows dynamic_conv1d_forward (DynamicConv1D.swift:358-401: loops ic then k, bias last)
    and conv1d_forward (Conv1D.swift:310-512); mode "reflect" pads as DynamicConv1D.swift:288-324,
    "zeros" as the shaders' bounds test. Input [C, L] or [B, C, L]."""
    x = _as(x, dtype)
    w = _as(w, dtype)
    squeeze = x.ndim == 2
    if squeeze:
        x = x[None]
    B, Cin, L = x.shape
    Cout, cinpg, K = w.shape
    if mode == "reflect":
        xp = reflect_pad(x, padding)
    else:
        xp = np.pad(x, ((0, 0), (0, 0), (padding, padding)))
    eff = (K - 1) * dilation + 1
    Lout = (xp.shape[-1] - eff) // stride + 1
    coutpg = Cout // groups
    y = np.empty((B, Cout, Lout), dtype=dtype)
    # window view [B, Cin, Lout, K]
    win = np.lib.stride_tricks.sliding_window_view(xp, eff, axis=-1)[..., ::stride, ::dilation]
    win = win[:, :, :Lout, :]
    for g in range(groups):
        xs = win[:, g * cinpg:(g + 1) * cinpg]                      # [B, cinpg, Lout, K]
        cols = np.ascontiguousarray(xs.transpose(0, 2, 1, 3)).reshape(B, Lout, cinpg * K)
        wg = w[g * coutpg:(g + 1) * coutpg].reshape(coutpg, cinpg * K)
        y[:, g * coutpg:(g + 1) * coutpg] = (cols @ wg.T).transpose(0, 2, 1)
    if b is not None:
        y += _as(b, dtype)[None, :, None]
    return y[0] if squeeze else y


def group_norm(x, num_groups, gamma=None, beta=None, eps=1e-5, dtype=np.float64):
    """Per (batch, group): mean, biased variance over C/G * L; y = gamma*(x-mean)/sqrt(var+eps)+beta.
    Follows GroupNorm.forwardCPU (Normalization.swift:665-724)."""
    x = _as(x, dtype)
    squeeze = x.ndim == 2
    if squeeze:
        x = x[None]
    B, C, L = x.shape
    xg = x.reshape(B, num_groups, -1)
    mean = xg.mean(axis=-1, keepdims=True)
    var = ((xg - mean) ** 2).mean(axis=-1, keepdims=True)
    inv = 1.0 / np.sqrt(var + eps)
    y = ((xg - mean) * inv).reshape(B, C, L)
    if gamma is not None:
        y = y * _as(gamma, dtype)[None, :, None] + _as(beta, dtype)[None, :, None]
    return y[0] if squeeze else y


def layer_norm(x, gamma=None, beta=None, eps=1e-5, dtype=np.float64):
    """Per row of the last axis: two-pass mean / biased variance, rsqrt(var + eps), affine.
    Follows layer_norm_forward (Normalization.swift:804-879)."""
    x = _as(x, dtype)
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + eps)
    if gamma is not None:
        y = y * _as(gamma, dtype) + _as(beta, dtype)
    return y


def gelu_tanh(x, dtype=np.float64):
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), the GELU of UNet.swift:118-131 and
    Transformer.swift:154-158."""
    x = _as(x, dtype)
    return 0.5 * x * (1.0 + np.tanh(SQRT_2_OVER_PI * (x + 0.044715 * x ** 3)))


def gelu_layer(x, dtype=np.float64):
    """GELU layer kernel (Activations.swift:124-137): clamp to [-10, 10] for the formula,
    x > 10 -> x, x < -10 -> 0."""
    x = _as(x, dtype)
    c = np.clip(x, -10.0, 10.0)
    r = 0.5 * c * (1.0 + np.tanh(SQRT_2_OVER_PI * (c + 0.044715 * c ** 3)))
    return np.where(x > 10.0, x, np.where(x < -10.0, 0.0, r))


def stable_sigmoid(x, dtype=np.float64):
    """Shaders/NN.metal:32-47: clamp to [-88, 88], 1/(1+e^-x) for x >= 0, e^x/(1+e^x) else."""
    x = np.clip(_as(x, dtype), -88.0, 88.0)
    pos = 1.0 / (1.0 + np.exp(-x))
    ex = np.exp(x)
    neg = ex / (1.0 + ex)
    return np.where(x >= 0.0, pos, neg)


def glu(x, axis=-2, dtype=np.float64):
    """out = a * sigmoid(b), a the first and b the second half along `axis`
    (glu kernel, Shaders/NN.metal:1012-1023: input[id] * stable_sigmoid(input[id + size]))."""
    x = _as(x, dtype)
    a, b = np.split(x, 2, axis=axis)
    return a * stable_sigmoid(b, dtype)


def activation(x, act: str, dtype=np.float64, alpha=0.01):
    """apply_activation of FusedConv1D / FusedLinear (Conv1D.swift:960-973, Linear.swift:630-639);
    alpha = leakyReluAlpha (default 0.01, Conv1D.swift:786)."""
    x = _as(x, dtype)
    if act == "none":
        return x
    if act == "relu":
        return np.maximum(x, 0.0)
    if act == "leaky_relu":
        return np.where(x >= 0.0, x, alpha * x)
    if act == "gelu":
        return gelu_tanh(x, dtype)
    if act == "swish":
        return x * stable_sigmoid(x, dtype)
    if act == "sigmoid":
        return stable_sigmoid(x, dtype)
    if act == "tanh":
        return np.tanh(x)
    raise ValueError(act)


def fused_conv1d(x, w, b=None, stride=1, padding=0, dilation=1, groups=1, act="none",
                 alpha=0.01, residual=None, dtype=np.float64):
    """FusedConv1D.forwardWithResidual (Conv1D.swift:857-900; kernel :975-1025): zero-padded
    conv + bias, then the activation, then the residual (added after the activation,
    :1016-1023)."""
    y = activation(conv1d(x, w, b, stride=stride, padding=padding, dilation=dilation,
                          groups=groups, dtype=dtype), act, dtype, alpha)
    return y if residual is None else y + _as(residual, dtype)


def linear(x, w, b=None, act="none", dtype=np.float64, alpha=0.01):
    """y = act(x W^T + b), W [out, in] (Linear.swift:337-365; linear_fused_forward :641-670);
    alpha = FusedLinear's leakyReluAlpha (Linear.swift:495)."""
    y = _as(x, dtype) @ _as(w, dtype).T
    if b is not None:
        y = y + _as(b, dtype)
    return activation(y, act, dtype, alpha)


def _softmax_ref(s):
    """Row softmax as Attention.swift:927-945: exp(s - max) / (sum + 1e-10)."""
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    return e / (e.sum(axis=-1, keepdims=True) + 1e-10)


def mha(xq, xkv, in_w, in_b, out_w, out_b, num_heads, dtype=np.float64):
    """MultiHeadAttention forward, following forwardCPU (Attention.swift:840-976):
    Q = xq Wq^T + bq, K = xkv Wk^T + bk, V = xkv Wv^T + bv with in_proj rows Q;K;V; head h uses
    columns [h*hd, (h+1)*hd); P = softmax(Q_h K_h^T / sqrt(hd)); O[:, h*hd+d]; out = O Wo^T + bo.
    xq [Sq, E] or [B, Sq, E]; xkv likewise (None = self-attention)."""
    xq = _as(xq, dtype)
    xkv = xq if xkv is None else _as(xkv, dtype)
    in_w = _as(in_w, dtype)
    out_w = _as(out_w, dtype)
    squeeze = xq.ndim == 2
    if squeeze:
        xq, xkv = xq[None], xkv[None]
    E = xq.shape[-1]
    hd = E // num_heads
    scale = 1.0 / np.sqrt(hd)
    bq = bk = bv = bo = None
    if in_b is not None:
        in_b = _as(in_b, dtype)
        bq, bk, bv = in_b[:E], in_b[E:2 * E], in_b[2 * E:]
    q = xq @ in_w[:E].T + (bq if bq is not None else 0.0)
    k = xkv @ in_w[E:2 * E].T + (bk if bk is not None else 0.0)
    v = xkv @ in_w[2 * E:].T + (bv if bv is not None else 0.0)
    B, Sq = q.shape[0], q.shape[1]
    o = np.empty_like(q)
    for bi in range(B):
        for h in range(num_heads):
            cs = slice(h * hd, (h + 1) * hd)
            s = (q[bi, :, cs] @ k[bi, :, cs].T) * scale
            o[bi, :, cs] = _softmax_ref(s) @ v[bi, :, cs]
    out = o @ out_w.T
    if out_b is not None:
        out = out + _as(out_b, dtype)
    return out[0] if squeeze else out


def feed_forward(x, w1, b1, w2, b2, dtype=np.float64):
    """Linear1 -> tanh-GELU -> Linear2 (FeedForward.forwardCPU, Transformer.swift:315-363)."""
    h = gelu_tanh(linear(x, w1, b1, dtype=dtype), dtype)
    return linear(h, w2, b2, dtype=dtype)


def encoder_block(x, conv_w, conv_b, norm_w, norm_b, num_groups, kernel_size=8, stride=4,
                  rewrite_w=None, rewrite_b=None, dtype=np.float64):
    """UNetEncoderBlock.forward (UNet.swift:80-100): DynamicConv1D with reflect padding
    (k-1)//2 (UNet.swift:52) -> GroupNorm -> tanh-GELU; with a rewrite weight [2C, C, 1], then
    the 1x1 conv C -> 2C and GLU over channels (NN.metal:1012-1023)."""
    pad = (kernel_size - 1) // 2
    y = conv1d(x, conv_w, conv_b, stride=stride, padding=pad, mode="reflect", dtype=dtype)
    y = gelu_tanh(group_norm(y, num_groups, norm_w, norm_b, dtype=dtype), dtype)
    if rewrite_w is None:
        return y
    z = conv1d(y, rewrite_w, rewrite_b, stride=1, padding=0, dtype=dtype)
    return glu(z, axis=-2, dtype=dtype)


def time_encoder(x, levels, dtype=np.float64):
    """Chained encoder levels composed in program order (each level sees the previous level's
    real output)."""
    y = _as(x, dtype)
    for lv in levels:
        y = encoder_block(y, lv["conv.weight"], lv["conv.bias"], lv["norm.weight"],
                          lv["norm.bias"], 1, rewrite_w=lv["rewrite.weight"],
                          rewrite_b=lv["rewrite.bias"], dtype=dtype)
    return y


def conv_transpose1d_length(L, kernel_size, stride=1, padding=0, output_padding=0, dilation=1):
    """outputLength(for:) (DynamicConv1D.swift:483-487)."""
    return (L - 1) * stride - 2 * padding + dilation * (kernel_size - 1) + output_padding + 1


def conv_transpose1d(x, w, b=None, stride=1, padding=0, output_padding=0, dilation=1, groups=1,
                     dtype=np.float64):
    """Transposed conv in scatter form: every input sample i of channel ic adds
    x[ic][i] * W[ic][oc][k] to output o = i*stride - padding + k*dilation (kept when
    0 <= o < Lout); weights [Cin, Cout/groups, K]. The same sum as the reference's per-output
    gather (dynamic_conv_transpose1d_forward, DynamicConv1D.swift:588-640), organised per tap k so
    each tap is one matrix product. Input [C, L] or [B, C, L]."""
    x = _as(x, dtype)
    w = _as(w, dtype)
    squeeze = x.ndim == 2
    if squeeze:
        x = x[None]
    B, Cin, L = x.shape
    cin_w, coutpg, K = w.shape
    assert cin_w == Cin and Cin % groups == 0
    Cout = coutpg * groups
    cinpg = Cin // groups
    Lout = conv_transpose1d_length(L, K, stride, padding, output_padding, dilation)
    y = np.zeros((B, Cout, Lout), dtype=dtype)
    i = np.arange(L)
    for g in range(groups):
        xg = x[:, g * cinpg:(g + 1) * cinpg]                      # [B, cinpg, L]
        for k in range(K):
            o = i * stride - padding + k * dilation
            keep = (o >= 0) & (o < Lout)
            if not keep.any():
                continue
            contrib = np.einsum("bcl,co->bol", xg[:, :, keep], w[g * cinpg:(g + 1) * cinpg, :, k],
                                optimize=True)
            y[:, g * coutpg:(g + 1) * coutpg][:, :, o[keep]] += contrib
    if b is not None:
        y += _as(b, dtype)[None, :, None]
    return y[0] if squeeze else y


def conv_transpose1d_gather(x, w, b=None, stride=1, padding=0, output_padding=0, dilation=1,
                            groups=1, dtype=np.float64):
    """The reference kernel's loop, one output at a time (DynamicConv1D.swift:588-640: ic, then k,
    input i = (o + padding - k*dilation) / stride when exact and in range, bias last). Pure Python:
    for small cases only (it pins conv_transpose1d)."""
    x = _as(x, dtype)
    w = _as(w, dtype)
    C, L = x.shape
    _, coutpg, K = w.shape
    Cout = coutpg * groups
    cinpg = C // groups
    Lout = conv_transpose1d_length(L, K, stride, padding, output_padding, dilation)
    y = np.zeros((Cout, Lout), dtype=dtype)
    for oc in range(Cout):
        g, ocg = divmod(oc, coutpg)
        for o in range(Lout):
            acc = 0.0
            for icg in range(cinpg):
                ic = g * cinpg + icg
                for k in range(K):
                    num = o + padding - k * dilation
                    if num >= 0 and num % stride == 0 and num // stride < L:
                        acc += x[ic, num // stride] * w[ic, ocg, k]
            y[oc, o] = acc + (b[oc] if b is not None else 0.0)
    return y


def decoder_block(x, skip, convt_w, convt_b, norm_w, norm_b, num_groups, kernel_size=8, stride=4,
                  dtype=np.float64):
    """UNetDecoderBlock.forward (UNet.swift:262-280): concat over channels (input first, then
    skip, UNet.swift:303-331) -> ConvTranspose1D with padding (k-1)//2 and output_padding
    stride - 2 + k % 2 (UNet.swift:229-241) -> GroupNorm -> tanh-GELU."""
    z = np.concatenate([_as(x, dtype), _as(skip, dtype)], axis=-2)
    y = conv_transpose1d(z, convt_w, convt_b, stride=stride, padding=(kernel_size - 1) // 2,
                         output_padding=stride - 2 + kernel_size % 2, dtype=dtype)
    return gelu_tanh(group_norm(y, num_groups, norm_w, norm_b, dtype=dtype), dtype)


def unet_padding(input_length, levels, kernel_size=8, stride=4):
    """UNetPaddingCalculator.calculatePadding (UNet.swift:393-430): pad to a multiple of
    stride**levels, half (rounded down) on the left."""
    divisor = stride ** levels
    rem = input_length % divisor
    if rem == 0:
        return 0, 0, input_length
    total = divisor - rem
    return total // 2, total - total // 2, input_length + total


def unet_bottleneck_length(input_length, levels, stride=4):
    """UNetPaddingCalculator.bottleneckLength (UNet.swift:432-447)."""
    for _ in range(levels):
        input_length //= stride
    return input_length


def time_unet(x, enc_levels, dec_levels, enc_groups=1, dtype=np.float64):
    """HTDemucs.forwardTimeUNet (HTDemucs.swift:521-548): the encoder chain keeps each level's
    output as its skip; decoder i takes the running signal and the skip of encoder level
    n-1-i. Encoder levels are the rewrite blocks of encoder_block; dec_levels hold
    conv_tr.weight / conv_tr.bias / norm.weight / norm.bias / groups."""
    y = _as(x, dtype)
    skips = []
    for lv in enc_levels:
        y = encoder_block(y, lv["conv.weight"], lv["conv.bias"], lv["norm.weight"],
                          lv["norm.bias"], enc_groups, rewrite_w=lv.get("rewrite.weight"),
                          rewrite_b=lv.get("rewrite.bias"), dtype=dtype)
        skips.append(y)
    for i, dv in enumerate(dec_levels):
        y = decoder_block(y, skips[len(skips) - 1 - i], dv["conv_tr.weight"], dv["conv_tr.bias"],
                          dv["norm.weight"], dv["norm.bias"], dv["groups"], dtype=dtype)
    return y


def _attn_args(p, pre):
    return (p[pre + "in_proj_weight"], p.get(pre + "in_proj_bias"), p[pre + "out_proj_weight"],
            p.get(pre + "out_proj_bias"))


def transformer_layer(x, p, num_heads, layer_scale=0.0, dtype=np.float64):
    """Pre-norm layer: y = x + g1*MHA(LN1 x); z = y + g2*FFN(LN2 y) (Transformer.swift:467-495
    sub-blocks 1 and 5; LayerScale g = layer_scale when > 0, else 1)."""
    x = _as(x, dtype)
    g1 = p.get("gamma_1.scale", layer_scale if layer_scale > 0 else 1.0)
    g2 = p.get("gamma_2.scale", layer_scale if layer_scale > 0 else 1.0)
    h = layer_norm(x, p["norm1.weight"], p["norm1.bias"], dtype=dtype)
    y = x + _as(g1, dtype) * mha(h, None, *_attn_args(p, "attn."), num_heads, dtype=dtype)
    h = layer_norm(y, p["norm2.weight"], p["norm2.bias"], dtype=dtype)
    ff = feed_forward(h, p["linear1.weight"], p["linear1.bias"], p["linear2.weight"],
                      p["linear2.bias"], dtype=dtype)
    return y + _as(g2, dtype) * ff


def cross_transformer(time, freq, p, num_layers, num_heads, dtype=np.float64):
    """Cross-domain bottleneck, HTDemucs layer structure: layer i even -> self-attention per
    branch; odd -> cross-attention where time attends to freq and freq to time, both reading the
    other branch's state from before the layer. Per branch:
    self : x += g1*MHA(LN1 x);           x += g2*FFN(LN2 x)
    cross: x += g1*MHA(LN1 x, LN2 other); x += g2*FFN(LN3 x)."""
    T = _as(time, dtype)
    F = _as(freq, dtype)

    def ln(x, pre):
        return layer_norm(x, p[pre + ".weight"], p[pre + ".bias"], dtype=dtype)

    def ffn(x, pre):
        return feed_forward(x, p[pre + "linear1.weight"], p[pre + "linear1.bias"],
                            p[pre + "linear2.weight"], p[pre + "linear2.bias"], dtype=dtype)

    for i in range(num_layers):
        pt, pf = f"layers.{i}.time.", f"layers.{i}.freq."
        if i % 2 == 0:
            new = []
            for X, pre in ((T, pt), (F, pf)):
                X = X + _as(p[pre + "gamma_1.scale"], dtype) * mha(
                    ln(X, pre + "norm1"), None, *_attn_args(p, pre + "attn."), num_heads, dtype)
                X = X + _as(p[pre + "gamma_2.scale"], dtype) * ffn(ln(X, pre + "norm2"), pre)
                new.append(X)
            T, F = new
        else:
            Tn = T + _as(p[pt + "gamma_1.scale"], dtype) * mha(
                ln(T, pt + "norm1"), ln(F, pt + "norm2"), *_attn_args(p, pt + "attn."),
                num_heads, dtype)
            Fn = F + _as(p[pf + "gamma_1.scale"], dtype) * mha(
                ln(F, pf + "norm1"), ln(T, pf + "norm2"), *_attn_args(p, pf + "attn."),
                num_heads, dtype)
            Tn = Tn + _as(p[pt + "gamma_2.scale"], dtype) * ffn(ln(Tn, pt + "norm3"), pt)
            Fn = Fn + _as(p[pf + "gamma_2.scale"], dtype) * ffn(ln(Fn, pf + "norm3"), pf)
            T, F = Tn, Fn
    return T, F


def cross_transformer_metalnn(time, freq, p, num_layers, num_heads, dtype=np.float64):
    """CrossTransformerEncoder with the reference class's own layer structure: the encoder runs
    its layers in order (Transformer.swift:626-667; the copies between layers are plain copies),
    each layer being TransformerLayer.forward(timeInput:freqInput:...) (:441-498), one
    addResidual per sub-block (:467-495):
      1. T += SA_t(LN_ts T) (:467-470);
      2. F += SA_f(LN_fs F);
      3. tn = LN_tc T, fn = LN_fc F; T += CA_t(tn, fn);
      4. F += CA_f(fn, tn) (tn from before step 3's update);
      5. T += FFN_t(LN_tf T); 6. F += FFN_f(LN_ff F).
    No LayerScale. Names as TransformerLayer.loadWeights (:529-557)."""
    T = _as(time, dtype)
    F = _as(freq, dtype)

    def ln(x, pre):
        return layer_norm(x, p[pre + ".weight"], p[pre + ".bias"], dtype=dtype)

    def ffn(x, pre):
        return feed_forward(x, p[pre + ".linear1.weight"], p[pre + ".linear1.bias"],
                            p[pre + ".linear2.weight"], p[pre + ".linear2.bias"], dtype=dtype)

    def attn(q, kv, pre):  # SafeTensorsLoader.loadAttentionWeights names (:335-339)
        return mha(q, kv, p[pre + ".in_proj_weight"], p[pre + ".in_proj_bias"],
                   p[pre + ".out_proj.weight"], p[pre + ".out_proj.bias"], num_heads, dtype)

    for i in range(num_layers):
        L = f"layers.{i}."
        T = T + attn(ln(T, L + "norm_time_self"), None, L + "self_attn_time")
        F = F + attn(ln(F, L + "norm_freq_self"), None, L + "self_attn_freq")
        tn = ln(T, L + "norm_time_cross")
        fn = ln(F, L + "norm_freq_cross")
        T = T + attn(tn, fn, L + "cross_attn_time")
        F = F + attn(fn, tn, L + "cross_attn_freq")
        T = T + ffn(ln(T, L + "norm_time_ffn"), L + "ffn_time")
        F = F + ffn(ln(F, L + "norm_freq_ffn"), L + "ffn_freq")
    return T, F


# ---------------------------------------------------------------- frequency branch (2-D)

def reflect_index(i, n):
    """Mirrored source index of padded position i - pad (applyReflectPadding2D,
    DynamicConv2D.swift:441-470): i < 0 -> -i, i >= n -> 2n - i - 2, then clamped to [0, n)."""
    i = np.asarray(i)
    i = np.where(i < 0, -i, i)
    i = np.where(i >= n, 2 * n - i - 2, i)
    return np.clip(i, 0, n - 1)


def conv2d_padding(H, W, kernel, stride, mode, pad, dilation):
    """computePadding (DynamicConv2D.swift:212-238)."""
    (kh, kw), (sh, sw), (dh, dw) = kernel, stride, dilation
    if mode == "valid":
        return 0, 0
    if mode == "same":
        ekh, ekw = (kh - 1) * dh + 1, (kw - 1) * dw + 1
        oh, ow = -(-H // sh), -(-W // sw)
        return max(0, (oh - 1) * sh + ekh - H) // 2, max(0, (ow - 1) * sw + ekw - W) // 2
    return pad


def conv2d_output_size(H, W, kernel, stride=(1, 1), mode="valid", pad=(0, 0), dilation=(1, 1)):
    """outputSize(forHeight:width:) (DynamicConv2D.swift:193-205)."""
    ph, pw = conv2d_padding(H, W, kernel, stride, mode, pad, dilation)
    nh = H + 2 * ph - ((kernel[0] - 1) * dilation[0] + 1)
    nw = W + 2 * pw - ((kernel[1] - 1) * dilation[1] + 1)
    if nh < 0 or nw < 0:
        return 0, 0
    return nh // stride[0] + 1, nw // stride[1] + 1


def conv2d(x, w, b=None, stride=(1, 1), mode="valid", pad=(0, 0), dilation=(1, 1), groups=1,
           dtype=np.float64):
    """y[oc][oh][ow] = bias[oc] + sum_{icg,kh,kw} xp[ic][oh*sh + kh*dh][ow*sw + kw*dw] * W[oc][icg][kh][kw]
    over the padded input xp: zeros, or mirrored samples for mode "reflect" (the reference pads
    first and runs the conv unpadded, DynamicConv2D.swift:309-383 and dynamic_conv2d_forward
    :525-590). Input [C, H, W] or [B, C, H, W]; W is [Cout, Cin/groups, KH, KW]."""
    x = _as(x, dtype)
    w = _as(w, dtype)
    squeeze = x.ndim == 3
    if squeeze:
        x = x[None]
    B, Cin, H, W = x.shape
    Cout, cinpg, KH, KW = w.shape
    assert Cin == cinpg * groups and Cout % groups == 0
    ph, pw = conv2d_padding(H, W, (KH, KW), stride, mode, pad, dilation)
    Ho, Wo = conv2d_output_size(H, W, (KH, KW), stride, mode, pad, dilation)
    if mode == "reflect":
        ri = reflect_index(np.arange(H + 2 * ph) - ph, H)
        ci = reflect_index(np.arange(W + 2 * pw) - pw, W)
        xp = x[:, :, ri][:, :, :, ci]
    else:
        xp = np.pad(x, ((0, 0), (0, 0), (ph, ph), (pw, pw)))
    y = np.zeros((B, Cout, Ho, Wo), dtype=dtype)
    coutpg = Cout // groups
    for g in range(groups):
        xs = xp[:, g * cinpg:(g + 1) * cinpg]
        ws = w[g * coutpg:(g + 1) * coutpg]
        for kh in range(KH):
            for kw in range(KW):
                r0, c0 = kh * dilation[0], kw * dilation[1]
                patch = xs[:, :, r0:r0 + (Ho - 1) * stride[0] + 1:stride[0],
                           c0:c0 + (Wo - 1) * stride[1] + 1:stride[1]]
                y[:, g * coutpg:(g + 1) * coutpg] += np.einsum("bchw,oc->bohw", patch,
                                                              ws[:, :, kh, kw], optimize=True)
    if b is not None:
        y += _as(b, dtype)[None, :, None, None]
    return y[0] if squeeze else y


def conv_transpose2d(x, w, b=None, stride=(1, 1), padding=(0, 0), output_padding=(0, 0),
                     dilation=(1, 1), groups=1, dtype=np.float64):
    """Scatter form of dynamic_conv_transpose2d_forward (DynamicConv2D.swift:890-955): input
    sample (ih, iw) of channel ic adds x * W[ic][ocg][kh][kw] to output (ih*sh - ph + kh*dh,
    iw*sw - pw + kw*dw) when inside; output size from outputSize (:727-736). W is
    [Cin, Cout/groups, KH, KW]; input [C, H, W] or [B, C, H, W]."""
    x = _as(x, dtype)
    w = _as(w, dtype)
    squeeze = x.ndim == 3
    if squeeze:
        x = x[None]
    B, Cin, H, W = x.shape
    cin_w, coutpg, KH, KW = w.shape
    assert cin_w == Cin and Cin % groups == 0
    Cout, cinpg = coutpg * groups, Cin // groups
    (sh, sw), (ph, pw), (oph, opw), (dh, dw) = stride, padding, output_padding, dilation
    Ho = (H - 1) * sh - 2 * ph + dh * (KH - 1) + oph + 1
    Wo = (W - 1) * sw - 2 * pw + dw * (KW - 1) + opw + 1
    # full (uncropped) canvas, then crop the padding
    Hf = max((H - 1) * sh + dh * (KH - 1) + 1, ph + Ho)
    Wf = max((W - 1) * sw + dw * (KW - 1) + 1, pw + Wo)
    full = np.zeros((B, Cout, Hf, Wf), dtype=dtype)
    for g in range(groups):
        xs = x[:, g * cinpg:(g + 1) * cinpg]
        for kh in range(KH):
            for kw in range(KW):
                contrib = np.einsum("bchw,co->bohw", xs, w[g * cinpg:(g + 1) * cinpg, :, kh, kw],
                                    optimize=True)
                full[:, g * coutpg:(g + 1) * coutpg, kh * dh:kh * dh + (H - 1) * sh + 1:sh,
                     kw * dw:kw * dw + (W - 1) * sw + 1:sw] += contrib
    y = full[:, :, ph:ph + Ho, pw:pw + Wo].copy()
    if b is not None:
        y += _as(b, dtype)[None, :, None, None]
    return y[0] if squeeze else y


def freq_encoder_block(x, conv_w, conv_b, norm_w, norm_b, num_groups, kernel=(3, 3),
                       stride=(2, 2), dtype=np.float64):
    """FreqUNetEncoderBlock2D.forward (FreqUNet2D.swift:84-117): Conv2D with reflect padding
    ((k-1)//2 per axis, :52-64) -> GroupNorm over [C, H*W] -> tanh-GELU."""
    pad = ((kernel[0] - 1) // 2, (kernel[1] - 1) // 2)
    y = conv2d(x, conv_w, conv_b, stride=stride, mode="reflect", pad=pad, dtype=dtype)
    shp = y.shape
    y = y.reshape(shp[:-2] + (shp[-2] * shp[-1],))
    y = gelu_tanh(group_norm(y, num_groups, norm_w, norm_b, dtype=dtype), dtype)
    return y.reshape(shp)


def freq_decoder_block(x, skip, convt_w, convt_b, norm_w, norm_b, num_groups, kernel=(3, 3),
                       stride=(2, 2), dtype=np.float64):
    """FreqUNetDecoderBlock2D.forward (FreqUNet2D.swift:281-306): concat over channels ->
    ConvTranspose2D (padding (k-1)//2, output padding stride-1, :245-260) -> GroupNorm ->
    tanh-GELU."""
    cat = np.concatenate([_as(x, dtype), _as(skip, dtype)], axis=-3)
    pad = ((kernel[0] - 1) // 2, (kernel[1] - 1) // 2)
    y = conv_transpose2d(cat, convt_w, convt_b, stride=stride, padding=pad,
                         output_padding=(stride[0] - 1, stride[1] - 1), dtype=dtype)
    shp = y.shape
    y = y.reshape(shp[:-2] + (shp[-2] * shp[-1],))
    y = gelu_tanh(group_norm(y, num_groups, norm_w, norm_b, dtype=dtype), dtype)
    return y.reshape(shp)


def unet_padding_2d(H, W, levels, stride):
    """UNetPaddingCalculator2D.calculatePadding (FreqUNet2D.swift:471-497)."""
    div = stride ** levels
    th = 0 if H % div == 0 else div - H % div
    tw = 0 if W % div == 0 else div - W % div
    return th // 2, th - th // 2, tw // 2, tw - tw // 2, H + th, W + tw
