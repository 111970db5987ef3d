"""Converts the reference's committed fixtures into compact .npz data files.

Sources (zkeown/MetalAudio Tests/MetalNNTests/Resources):
* HTDemucsReference/time_encoder_level{0,1}.json (scripts/generate_htdemucs_reference.py:40-96:
  Conv1d with reflect padding (k-1)//2, xavier-uniform weights, zero bias, GroupNorm(8),
  tanh-GELU; HTDemucsValidationTests.swift:37-117, abs 1e-4 or rel 1e-3);
* HTDemucsReference/freq_encoder_level{0,1}.json (generate_htdemucs_reference.py:99-160: Conv2d
  3x3 stride 2 with reflect padding 1, GroupNorm(8), tanh-GELU);
* Conv2DReference/*.json (PyTorch Conv2d / ConvTranspose2d with zero padding; checked by
  Conv2DValidationTests.swift at abs 1e-4 / rel 1e-3).
Only the data arrays are kept (inputs, weights, expected outputs, shapes, config), stored as
float32 / int64.

Run in a container that has /root/reference: python tests/golden/make_fixtures.py
"""
import json
import sys
from pathlib import Path

import numpy as np

RES = Path("/root/reference/Tests/MetalNNTests/Resources")
SRC = RES / "HTDemucsReference"
OUT = Path(__file__).resolve().parent


def convert(name: str) -> None:
    d = json.loads((SRC / f"{name}.json").read_text())
    cfg = d["config"]
    cin, cout, k = cfg["in_channels"], cfg["out_channels"], cfg["kernel_size"]
    in_shape = tuple(d["input_shape"])
    out_shape = tuple(d["output_shape"])
    np.savez_compressed(
        OUT / f"{name}.npz",
        input=np.asarray(d["input"], np.float32).reshape(in_shape),
        conv_weight=np.asarray(d["conv_weight"], np.float32).reshape(cout, cin, k),
        conv_bias=np.asarray(d["conv_bias"], np.float32),
        norm_weight=np.asarray(d["norm_weight"], np.float32),
        norm_bias=np.asarray(d["norm_bias"], np.float32),
        output=np.asarray(d["output"], np.float32).reshape(out_shape),
        config=np.asarray([cin, cout, k, cfg["stride"], cfg["num_groups"]], np.int64),
    )
    print(f"{name}: input {in_shape} -> output {out_shape}")


def convert_freq(name: str) -> None:
    d = json.loads((SRC / f"{name}.json").read_text())
    cfg = d["config"]
    cin, cout = cfg["in_channels"], cfg["out_channels"]
    kh, kw = cfg["kernel_size"]
    np.savez_compressed(
        OUT / f"{name}.npz",
        input=np.asarray(d["input"], np.float32).reshape(d["input_shape"]),
        conv_weight=np.asarray(d["conv_weight"], np.float32).reshape(cout, cin, kh, kw),
        conv_bias=np.asarray(d["conv_bias"], np.float32),
        norm_weight=np.asarray(d["norm_weight"], np.float32),
        norm_bias=np.asarray(d["norm_bias"], np.float32),
        output=np.asarray(d["output"], np.float32).reshape(d["output_shape"]),
        config=np.asarray([cin, cout, kh, kw, *cfg["stride"], cfg["num_groups"]], np.int64),
    )
    print(f"{name}: input {d['input_shape']} -> output {d['output_shape']}")


def convert_conv2d() -> None:
    """All Conv2DReference cases into one archive: <case>/<array>."""
    arrays = {}
    for f in sorted((RES / "Conv2DReference").glob("*.json")):
        d = json.loads(f.read_text())
        if "name" not in d:
            continue
        cfg = d["config"]
        n = d["name"]
        arrays[f"{n}/input"] = np.asarray(d["input"], np.float32).reshape(d["input_shape"])
        arrays[f"{n}/weight"] = np.asarray(d["weight"], np.float32).reshape(d["weight_shape"])
        arrays[f"{n}/output"] = np.asarray(d["output"], np.float32).reshape(d["output_shape"])
        if d.get("bias") is not None:
            arrays[f"{n}/bias"] = np.asarray(d["bias"], np.float32)
        arrays[f"{n}/config"] = np.asarray(
            [cfg["in_channels"], cfg["out_channels"], *cfg["kernel_size"], *cfg["stride"],
             *cfg["padding"], *cfg.get("output_padding", [0, 0]), *cfg["dilation"],
             cfg["groups"], int("output_padding" in cfg)], np.int64)
        print(f"Conv2DReference/{n}: {d['input_shape']} -> {d['output_shape']}")
    np.savez_compressed(OUT / "conv2d_reference.npz", **arrays)


if __name__ == "__main__":
    if not SRC.exists():
        sys.exit(f"{SRC} not found")
    for n in ("time_encoder_level0", "time_encoder_level1"):
        convert(n)
    for n in ("freq_encoder_level0", "freq_encoder_level1"):
        convert_freq(n)
    convert_conv2d()
