"""Host-side logic on the CPU: torch weight preparation against the oracle,
the Python geometry mirror, op schemas and fake kernels, and the refusal to
run on CPU tensors (there is no CPU fallback)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import w4a8 as ow


@pytest.mark.parametrize("K,G", [(5120, 128), (1024, 64), (1057, 128), (100, 33), (33, 64), (777, 96)])
def test_geometry_mirror(pkg, K, G):
    g = pkg.geometry
    assert g.num_groups(K, G) == ow.num_groups(K, G)
    assert g.kpad(K, G) == ow.kpad(K, G)
    assert all(g.group_real(i, K, G) == ow.group_real(i, K, G) for i in range(g.num_groups(K, G)))


@pytest.mark.parametrize("N,K,G", [(64, 1024, 128), (48, 512, 64), (32, 1057, 128), (16, 100, 33)])
def test_quantize_weight_matches_oracle(pkg, N, K, G):
    rng = np.random.default_rng(N + K)
    w = rng.standard_normal((N, K)).astype(np.float32)
    w[0, :5] = 0.0
    w[1, :] = 0.0                                  # an all-zero row -> tiny scales
    wt = torch.from_numpy(w).to(torch.bfloat16)
    w_q, w_scale = pkg.packing.quantize_weight(wt, G)
    codes, scales = ow.quantize_weight_sym(wt.float().numpy(), G)
    assert np.array_equal(w_q.numpy(), ow.pack_grouped(codes, G))
    assert np.array_equal(w_scale.view(torch.int16).numpy().view(np.uint16), scales.T)
    if K % 2 == 0:
        rt = pkg.packing.unpack_int4(pkg.packing.pack_int4(torch.from_numpy(codes)))
        assert np.array_equal(rt.numpy(), codes)


def test_synthetic_distributions(pkg):
    s = pkg.synth
    x = s.bf16_bits_to_f32(s.activations(64, 5120, 0))
    big = np.abs(x).max(axis=0) > 8
    assert 3 <= big.sum() <= 8                      # ~5 outlier channels of 5120
    w = s.weight_codes_uniform(64, 512, 1)
    assert w.min() == -8 and w.max() == 7
    sc = s.scale_bits_to_f32(s.group_scales(64, 4, 2, "f16"), "f16")
    assert sc.min() >= 0.0019 and sc.max() <= 0.0201


def test_fake_kernels_give_shapes(pkg):
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty((5, 1024), dtype=torch.bfloat16, device="cuda")
        a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x)
        assert a_q.shape == (5, 1024) and a_q.dtype == torch.int8 and a_s.shape == (5,)
        # with a ragged group geometry the quant output is the padded layout
        x2 = torch.empty((5, 1057), dtype=torch.bfloat16, device="cuda")
        assert torch.ops.npu.w4a8_quant_pertoken(x2, 1024)[0].shape == (5, 1088)
        w_q = torch.empty((300, 512), dtype=torch.int8, device="cuda")
        ws = torch.empty((8, 300), dtype=torch.float16, device="cuda")
        wt, st = torch.ops.npu.w4a8_repack(w_q, ws, 1024, 128)
        assert wt.numel() == 19 * 8 * 1024 and tuple(st.shape) == (19, 8, 16)
        y = torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, 300, 1024, 128)
        assert y.shape == (5, 300) and y.dtype == torch.bfloat16
        y2, P = torch.ops.npu.w4a8_gemm_partials(a_q, a_s, wt, st, 300, 1024, 128)
        assert P.shape == (8, 5, 300) and P.dtype == torch.int32


def test_cpu_tensors_are_refused(pkg):
    x = torch.zeros((2, 64), dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        torch.ops.npu.w4a8_quant_pertoken(x)


def test_quantize_weight_asym_matches_oracle(pkg):
    """The torch export (the reference's quantize_weight, asymmetric) and the oracle's
    restatement agree byte for byte, ragged tail and constant rows included."""
    from oracle import w4a8 as ow
    w = torch.randn(24, 1057, generator=torch.Generator().manual_seed(4)) * 0.03
    w[5] = 0.125
    w_q, ws, wk, wz = pkg.packing.quantize_weight_asym(w, 1024)
    codes, sc, zr, ks = ow.quantize_weight_asym(w.numpy(), 1024)
    assert np.array_equal(w_q.numpy(), ow.pack_grouped(codes, 1024))
    assert np.array_equal(ws.view(torch.int16).numpy().view(np.uint16), sc)
    assert np.array_equal(wz.view(torch.int16).numpy().view(np.uint16), zr)
    assert np.array_equal(wk.numpy(), ks)


def test_midgroup_fake_kernels_give_shapes(pkg):
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty((5, 1057), dtype=torch.bfloat16, device="cuda")
        a_hi, a_lo, a_s, a_k = torch.ops.npu.midgroup_quant_a(x)
        assert a_hi.shape == (16, 544) and a_s.shape == (2, 16) and a_k.dtype == torch.int32
        w_q = torch.empty((256, 544), dtype=torch.int8, device="cuda")
        gn = torch.empty((2, 256), dtype=torch.bfloat16, device="cuda")
        y = torch.ops.npu.midgroup_w4a8_gemm(a_hi, a_lo, a_s, a_k, w_q, gn, gn.int(), gn, 1057)
        assert y.shape == (16, 256) and y.dtype == torch.bfloat16



def _vendor_pack_n(codes: torch.Tensor) -> torch.Tensor:
    """Test-side packer: two int4 per byte along N, low nibble = even row."""
    c = codes.to(torch.int16) & 0xF
    return (c[0::2] | (c[1::2] << 4)).to(torch.uint8).view(torch.int8)


def test_vendor_w4a8_dynamic_conversion(pkg):
    g = torch.Generator().manual_seed(7)
    N, K, G = 64, 512, 128
    codes = torch.randint(-8, 8, (N, K), dtype=torch.int8, generator=g)
    s2 = (torch.rand((N, K // G), generator=g) * 0.01 + 0.001).to(torch.float16)
    base = "model.layers.0.mlp.down_proj"
    t = {f"{base}.weight": _vendor_pack_n(codes), f"{base}.weight_scale": torch.full((N, 1), 2.0),
         f"{base}.weight_offset": torch.zeros((N, 1)), f"{base}.weight_scale_second": s2,
         f"{base}.weight_offset_second": torch.zeros((N, K // G), dtype=torch.float16),
         f"{base}.scale_bias": torch.zeros((N, 16))}
    assert torch.equal(pkg.checkpoint.vendor_unpack_n(t[f"{base}.weight"]), codes)
    w_q, w_scale, n, k = pkg.checkpoint.vendor_to_grouped(t, base, G)
    assert (n, k) == (N, K)
    assert torch.equal(pkg.packing.unpack_int4(w_q), codes)
    assert torch.equal(w_scale, (2.0 * s2.float()).to(torch.float16).T)
    t[f"{base}.weight_offset"] = torch.ones((N, 1))
    with pytest.raises(ValueError, match="weight_offset"):
        pkg.checkpoint.vendor_to_grouped(t, base, G)


def test_midgroup_export_and_load_roundtrip(pkg, tmp_path):
    g = torch.Generator().manual_seed(8)
    src = {"model.layers.0.self_attn.o_proj.weight": torch.randn((96, 1057), generator=g) * 0.05,
           "model.norm.weight": torch.ones(1057)}
    out = pkg.checkpoint.export_midgroup(src, 1024)
    base = "model.layers.0.self_attn.o_proj"
    assert set(out) == {f"{base}.{s}" for s in pkg.checkpoint.MIDGROUP_SUFFIXES} | {"model.norm.weight"}
    wq, ws, wk, wz = pkg.packing.quantize_weight_asym(src[f"{base}.weight"].to(torch.bfloat16), 1024)
    assert torch.equal(out[f"{base}.weight_packed"], wq) and torch.equal(out[f"{base}.weight_scale"], ws.T)
    assert out[f"{base}.weight_ksum"].shape == (96, 2) and out[f"{base}.weight_zero"].dtype == torch.bfloat16
    from safetensors.torch import save_file
    save_file(out, str(tmp_path / "model-00001.safetensors"), metadata={"format": "pt"})
    out = pkg.checkpoint.load_safetensors(str(tmp_path / "model-00001.safetensors"))
    m = pkg.checkpoint.load_midgroup_linear(out, base, K=1057, device="cpu")
    assert torch.equal(m.weight_packed, wq) and torch.equal(m._gn[0], ws)
    with pytest.raises(ValueError):
        pkg.checkpoint.load_midgroup_linear(out, base, K=1100, device="cpu")
    assert pkg.checkpoint.quant_config(1024)["packed_layout"] == "mg_kgeom_v1"


# ------------------------------------------------------------------ vLLM-style linear methods
def test_vllm_plugin_configs_and_weights(pkg):
    """The quant-method contract without vLLM: config parsing, the parameters
    create_weights registers (checkpoint layout, output_dim 0, loader), the
    row-parallel refusal and the load-time transpose of the mid-group tensors."""
    vp = pkg.vllm_plugin
    cfg = vp.MidGroupW4A8Config.from_config({"quant_method": "midgroup_w4a8", "group_size": 1024, "sym": False})
    assert cfg.get_name() == "midgroup_w4a8" and cfg.group_size == 1024 and cfg.quant_description == {}
    assert cfg.get_supported_act_dtypes() == [torch.bfloat16]
    assert cfg.get_quant_method(torch.nn.Module(), "model.lm_head") is None
    m = cfg.get_quant_method(torch.nn.Module(), "model.layers.0.self_attn.o_proj")
    layer = torch.nn.Module()
    loader = object()
    m.create_weights(layer, 3456, [256, 128], 3456, 384, torch.bfloat16, weight_loader=loader)
    G = 4                      # 3456 = 3 full groups + a short one of 384
    assert tuple(layer.weight_packed.shape) == (384, pkg.geometry.kpad(3456, 1024) // 2)
    assert pkg.geometry.kpad(3456, 1024) == 3 * 1024 + 384
    for name, dt in (("weight_scale", torch.bfloat16), ("weight_zero", torch.bfloat16), ("weight_ksum", torch.int32)):
        t = getattr(layer, name)
        assert tuple(t.shape) == (384, G) and t.dtype == dt and t.output_dim == 0 and t.weight_loader is loader
        assert not t.requires_grad
    with torch.no_grad():
        layer.weight_scale.copy_(torch.arange(384 * G, dtype=torch.float32).reshape(384, G).to(torch.bfloat16))
    ref = layer.weight_scale.detach().clone()
    m.process_weights_after_loading(layer)
    assert tuple(layer.weight_scale.shape) == (G, 384) and torch.equal(layer.weight_scale, ref.t())
    with pytest.raises(ValueError, match="K-sharded"):
        m.create_weights(torch.nn.Module(), 2560, [5120], 5120, 5120, torch.bfloat16)

    pt = vp.PerTokenW4A8Config.from_config({"quant_method": "w4a8_pertoken", "group_size": 128,
                                             "scale_dtype": "bfloat16"})
    assert pt.get_name() == "w4a8_pertoken" and pt.scale_dtype == "bfloat16"
    layer2 = torch.nn.Module()
    pt.get_quant_method(layer2, "model.layers.0.mlp.down_proj").create_weights(
        layer2, 5120, [1024], 5120, 1024, torch.bfloat16)
    assert tuple(layer2.weight_packed.shape) == (1024, 2560) and layer2.weight_scale.dtype == torch.bfloat16
    assert tuple(layer2.weight_scale.shape) == (1024, 40)
    with pytest.raises(ValueError):
        vp.PerTokenW4A8Config(scale_dtype="float32")
    if not vp.HAVE_VLLM:
        with pytest.raises(ImportError):
            vp.register()
