"""The checkpoint reader (qwen3.8-27b-mlx_amd/weights.py) against a small checkpoint written
here in the reference's format: config.json (text_config + quantization) and two
safetensors shards with "model.language_model." names, 4-bit projections as mx.quantize
stores them (weight (N, K/8) uint32, scales and biases (N, K/64) bf16) and one projection
left in bf16 (cpp/src/model.cpp:85-104, 149-183, 266-340, 733-754)."""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

HK, HV, D, KC, H = 2, 6, 128, 4, 1024
QKV = 2 * HK * D + HV * D
Z = HV * D
PFX = "model.language_model.layers.0.linear_attn."


def write_checkpoint(path, rng, out_proj_quantized=False, drop=None, bad_shape=None,
                     hk=HK, hv=HV, cfg_override=None):
    import torch
    from safetensors.torch import save_file
    os.makedirs(path, exist_ok=True)
    t = {}
    QKV, Z, HV = 2 * hk * D + hv * D, hv * D, hv

    def bf16(*shape):
        return torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(torch.bfloat16)

    def quant(name, n, k):
        t[PFX + name + ".weight"] = torch.from_numpy(
            rng.integers(0, 2 ** 32, (n, k // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)).view(torch.uint32)
        t[PFX + name + ".scales"] = bf16(n, k // 64).abs() * 0.01
        t[PFX + name + ".biases"] = bf16(n, k // 64) * 0.1

    t[PFX + "conv1d.weight"] = bf16(QKV, 1, KC) * 0.1
    t[PFX + "A_log"] = bf16(HV)
    t[PFX + "dt_bias"] = bf16(HV) * 0.1
    t[PFX + "norm.weight"] = bf16(D) * 0.1 + 1.0
    quant("in_proj_qkv", QKV, H)
    quant("in_proj_z", Z, H)
    quant("in_proj_a", HV, H)
    quant("in_proj_b", HV, H)
    mods = [PFX + m for m in ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b")]
    if out_proj_quantized:
        quant("out_proj", H, Z)
        mods.append(PFX + "out_proj")
    else:
        t[PFX + "out_proj.weight"] = bf16(H, Z)
    if drop:
        del t[PFX + drop]
    if bad_shape:
        t[PFX + bad_shape] = bf16(3)
    names = sorted(t)
    half = len(names) // 2
    save_file({n: t[n].contiguous() for n in names[:half]}, os.path.join(path, "model-00001-of-00002.safetensors"))
    save_file({n: t[n].contiguous() for n in names[half:]}, os.path.join(path, "model-00002-of-00002.safetensors"))
    cfg = {"text_config": {"hidden_size": H, "num_hidden_layers": 2,
                           "layer_types": ["linear_attention", "full_attention"],
                           "linear_num_key_heads": hk, "linear_num_value_heads": hv,
                           "linear_key_head_dim": D, "linear_value_head_dim": D,
                           "linear_conv_kernel_dim": KC, "rms_norm_eps": 1e-6},
           "quantization": {"group_size": 64, "bits": 4, "quantized_modules": mods}}
    cfg["text_config"].update(cfg_override or {})
    json.dump(cfg, open(os.path.join(path, "config.json"), "w"))
    return t


def test_reader_layouts_and_values(gdn, tmp_path):
    import torch
    t = write_checkpoint(str(tmp_path), np.random.default_rng(1))
    ck = gdn.weights.Checkpoint(str(tmp_path))
    assert ck.config.hidden_size == H and ck.config.quantized and ck.config.layer_types[1] == "full_attention"
    L = ck.deltanet_layer(0, device="cpu")
    conv = t[PFX + "conv1d.weight"]
    assert L.conv_weight.dtype == torch.bfloat16 and tuple(L.conv_weight.shape) == (KC, QKV)
    assert torch.equal(L.conv_weight, conv[:, 0, :].t())            # w[j, c] = conv1d.weight[c, 0, j]
    assert L.A_log.dtype == torch.float32 and torch.equal(L.A_log, t[PFX + "A_log"].float())
    assert torch.equal(L.dt_bias, t[PFX + "dt_bias"].float())
    assert torch.equal(L.norm_gamma, t[PFX + "norm.weight"].float())  # not zero-centred
    for name in ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b"):
        q = getattr(L, name)
        assert isinstance(q, gdn.QuantLinear)
        assert torch.equal(q.w, t[PFX + name + ".weight"].view(torch.int32))
        assert torch.equal(q.scales, t[PFX + name + ".scales"])
        assert torch.equal(q.biases, t[PFX + name + ".biases"])
    assert L.in_proj_qkv.n == QKV and L.in_proj_a.n == HV
    assert isinstance(L.out_proj, gdn.weights.PlainLinear)
    assert torch.equal(L.out_proj.weight, t[PFX + "out_proj.weight"])
    assert list(ck.deltanet_layers(device="cpu")) == [0]


def test_reader_errors(gdn, tmp_path):
    rng = np.random.default_rng(2)
    write_checkpoint(str(tmp_path / "a"), rng, drop="dt_bias")
    with pytest.raises(KeyError, match="missing tensor 'layers.0.linear_attn.dt_bias'"):
        gdn.weights.Checkpoint(str(tmp_path / "a")).deltanet_layer(0, device="cpu")
    write_checkpoint(str(tmp_path / "b"), rng, bad_shape="A_log")
    with pytest.raises(ValueError, match="has shape"):
        gdn.weights.Checkpoint(str(tmp_path / "b")).deltanet_layer(0, device="cpu")
    write_checkpoint(str(tmp_path / "c"), rng)
    with pytest.raises(ValueError, match="full_attention"):
        gdn.weights.Checkpoint(str(tmp_path / "c")).deltanet_layer(1, device="cpu")


@pytest.mark.parametrize("override,msg", [
    (dict(linear_conv_kernel_dim=3), "linear_conv_kernel_dim = 3"),
    (dict(linear_key_head_dim=64), "head dims = 64/128"),
    (dict(linear_value_head_dim=256), "head dims = 128/256"),
    (dict(linear_num_value_heads=5), "not a multiple"),
])
def test_reader_rejects_shapes_the_kernels_do_not_take(gdn, tmp_path, override, msg):
    """A config the kernels cannot run (other conv taps, head dims, a fractional v-head to
    k-head ratio) is refused at load, before any tensor is read."""
    write_checkpoint(str(tmp_path), np.random.default_rng(3), cfg_override=override)
    with pytest.raises(ValueError, match=msg):
        gdn.weights.Checkpoint(str(tmp_path)).deltanet_layer(0, device="cpu")


@pytest.mark.gpu
def test_checkpoint_layer_through_the_kernels(O, gdn, dev, tmp_path):
    """One DeltaNet layer read from a checkpoint and run through the kernels at B=2, T=1
    (model.cpp:585-641): in_proj (4 matrices, one call), the conv + gates + recurrence step,
    then out_proj(GatedRMSNorm(o, z)). Each stage is checked against the oracle on the
    device's own inputs to that stage: the projections to the qlinear bound (2^-8 |y| plus
    the fp32 accumulation bound), o and the state to 1e-4."""
    import torch
    from _util import bf16_to_f32, log_case, to_dev, to_np
    from test_gpu_qlinear import bound, check
    log_case("checkpoint layer: Hk=4 Hv=8 hidden 1024, B=2 T=1")
    hk, hv, B = 4, 8, 2
    d = str(tmp_path)
    t = write_checkpoint(d, np.random.default_rng(3), out_proj_quantized=True, hk=hk, hv=hv)
    ck = gdn.weights.Checkpoint(d)
    L = ck.deltanet_layer(0, device=dev)

    def host(name):
        v = t[PFX + name]
        return v.view(torch.int32).numpy().view(np.uint32) if v.dtype == torch.uint32 else to_np(v)
    rng = np.random.default_rng(4)
    x = O.to_bf16(rng.standard_normal((B, H)).astype(np.float32))
    ys = gdn.qlinear([L.in_proj_qkv, L.in_proj_z, L.in_proj_a, L.in_proj_b], to_dev(x, dev))
    torch.cuda.synchronize()
    got = [to_np(y) for y in ys]
    for name, g in zip(("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b"), got):
        w, s, b = host(name + ".weight"), host(name + ".scales"), host(name + ".biases")
        check(g, O.qlinear(x, w, s, b), bound(O, x, s, b), name)
    qkv, z, a, b = got
    cache = gdn.DeltaCache(B, Hv=hv, Hk=hk, device=dev)
    o = cache.step(to_dev(qkv.reshape(B, 1, -1), dev), L.conv_weight, to_dev(a.reshape(B, 1, hv), dev),
                   to_dev(b.reshape(B, 1, hv), dev), L.A_log, L.dt_bias, o_dtype=torch.float32)
    torch.cuda.synchronize()
    inp = O.LayerInputs(None, None, None, qkv.reshape(B, 1, -1), to_np(L.conv_weight), None,
                        a.reshape(B, 1, hv), b.reshape(B, 1, hv), to_np(L.A_log), to_np(L.dt_bias),
                        None)
    ref = O.reference_layer(inp)
    o_np = to_np(o)
    assert O.rel_err(o_np, ref["o"]) <= 1e-4 and O.max_abs(o_np, ref["o"]) <= 1e-4
    assert O.rel_err(to_np(cache.state), ref["state"]) <= 1e-4
    (y,) = gdn.qlinear([L.out_proj], norm=(o.reshape(B, hv * D), to_dev(z, dev), L.norm_gamma, 1e-6))
    torch.cuda.synchronize()
    xn = O.gated_rmsnorm(o_np.reshape(B * hv, D), z.reshape(B * hv, D), to_np(L.norm_gamma),
                         1e-6).reshape(B, hv * D)
    w, s, b = host("out_proj.weight"), host("out_proj.scales"), host("out_proj.biases")
    W = np.abs(np.repeat(bf16_to_f32(s), 64, axis=1)) * 15 + np.abs(np.repeat(bf16_to_f32(b), 64, axis=1))
    flip = 3 * 2.0 ** -8 * (np.abs(bf16_to_f32(xn)).max(axis=1, keepdims=True) * W.max(axis=1)[None, :])
    check(to_np(y), O.qlinear(xn, w, s, b), bound(O, xn, s, b) + flip, "out_proj")
