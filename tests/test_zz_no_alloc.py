"""The allocation-free GroupNorm forward (mnn_groupnorm_forward_noalloc) against the allocating
entry point (mnn_layer_forward) through the C ABI: two calls in a row, the second smaller, each
bitwise equal to the allocating forward (same kernels) and within the fp32 bar of the oracle."""
import ctypes
import sys

import numpy as np
import pytest

import oracle
from metalaudio_amd import nn
from metalaudio_amd._lib import check, lib
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(97)


def say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def noalloc(layer, x, out, stream):
    check(lib().mnn_groupnorm_forward_noalloc(layer.handle, x.handle, out.handle, stream.handle))


def allocations():
    n = ctypes.c_int64()
    check(lib().mnn_debug_device_allocations(ctypes.byref(n)))
    return n.value


@pytest.mark.parametrize("G,act", [(1, "gelu"), (4, "none")])
def test_groupnorm_noalloc_matches_forward(G, act):
    dev = nn.AudioDevice(0)
    stream = nn.Stream(dev)
    C = 48
    gm = (1 + 0.2 * RNG.standard_normal(C)).astype(np.float32)
    bt = (0.2 * RNG.standard_normal(C)).astype(np.float32)
    layer = nn.GroupNorm(dev, G, C, activation=act)
    layer.load_parameters(gm, bt)
    for B, L in ((2, 85995), (1, 1000)):  # second call smaller: stale scratch must not leak in
        say(f"groupnorm noalloc G={G} act={act} B={B} L={L}")
        x = (RNG.standard_normal((B, C, L)) * 3 + 0.5).astype(np.float32)
        xt = nn.Tensor.from_numpy(dev, x)
        got, want = nn.Tensor(dev, x.shape), nn.Tensor(dev, x.shape)
        before = allocations()
        noalloc(layer, xt, got, stream)  # first call on a fresh layer: nothing may be reserved
        stream.sync(60000)
        assert allocations() == before
        layer.forward(xt, want, stream)
        stream.sync(60000)
        g = got.to_numpy()
        np.testing.assert_array_equal(g, want.to_numpy())
        assert_close(g, oracle.activation(oracle.group_norm(x, G, gm, bt), act), 1e-4, 1e-3,
                     "groupnorm noalloc")


def test_groupnorm_noalloc_rejects_oversize_and_other_layers():
    dev = nn.AudioDevice(0)
    stream = nn.Stream(dev)
    say("groupnorm noalloc limits")
    G = 32768  # one partial per (batch, group): 32768 > 21845 partials
    layer = nn.GroupNorm(dev, G, G)
    x = nn.Tensor(dev, (1, G, 1))
    with pytest.raises(nn.MNNError) as e:
        noalloc(layer, x, nn.Tensor(dev, (1, G, 1)), stream)
    assert e.value.name == "MNN_ERR_INVALID_CONFIGURATION" and "scratch" in str(e.value)
    lin = nn.Linear(dev, 4, 4)
    with pytest.raises(nn.MNNError) as e:
        noalloc(lin, nn.Tensor(dev, (4,)), nn.Tensor(dev, (4,)), stream)
    assert e.value.name == "MNN_ERR_INVALID_ARGUMENT"
    gn = nn.GroupNorm(dev, 1, 8)
    xb = nn.Tensor(dev, (1, 8, 64), dtype="bf16")  # 2-byte elements: would be read as 4-byte
    with pytest.raises(nn.MNNError) as e:
        noalloc(gn, xb, nn.Tensor(dev, (1, 8, 64)), stream)
    assert e.value.name == "MNN_ERR_INVALID_ARGUMENT"
