"""Config-5 GPT harness (helion_amd/gpt.py): parameter layout on the CPU, and
on the GPU the training step on the HIP kernel layer against its pure-PyTorch
twin from identical weights and batches (the loss-curve parity the benchmark
reports over 200 steps, here at a small size and 8 steps)."""

from __future__ import annotations

import pytest
import torch

from helion_amd import gpt


def test_config5_parameter_count():
    # 12 x (4 x 768^2 + 3 x 768 x 3072 + 2 x 768) + 50304 x 768 + 768, tied embeddings
    assert gpt.n_params(gpt.GPTConfig()) == 151_898_880


def test_init_is_seeded_and_shaped():
    cfg = gpt.GPTConfig(vocab_size=64, d_model=32, n_layers=2, n_heads=2, head_dim=16, d_ff=64)
    a, b = gpt.init_params(cfg, 0), gpt.init_params(cfg, 0)
    assert list(a) == [n for n, _ in gpt.param_shapes(cfg)]
    for k in a:
        assert torch.equal(a[k], b[k])
        assert a[k].dtype == torch.float32
    assert torch.equal(a["final_norm"], torch.ones(32))
    assert abs(float(a["embed"].std()) - 0.02) < 0.005


def test_split_k_choice():
    # the measured split counts at the config-5 shapes (16384 tokens); slices stay >= 512 tokens
    assert [gpt._split_k(o, i, 16384) for o, i in [(768, 768), (2304, 768), (768, 3072), (6144, 768)]] \
        == [16, 4, 4, 2]
    assert gpt._split_k(768, 768, 1024) == 2 and gpt._split_k(768, 768, 1000) == 1


@pytest.mark.gpu
@pytest.mark.parametrize(("n_out", "n_in"), [(768, 768), (2304, 768), (96, 40)])
def test_projection_split_k_gradients(n_out, n_in):
    # _Proj: the split-K weight gradient is the fp32-accumulated product rounded once
    g = torch.Generator().manual_seed(n_out)
    x = torch.randn(4096, n_in, generator=g).bfloat16().cuda().requires_grad_(True)
    w = (torch.randn(n_out, n_in, generator=g) * 0.02).bfloat16().cuda().requires_grad_(True)
    dy = torch.randn(4096, n_out, generator=g).bfloat16().cuda()
    y = gpt._Proj.apply(x, w)
    y.backward(dy)
    x32, w32, dy32 = x.detach().double().cpu(), w.detach().double().cpu(), dy.double().cpu()
    torch.testing.assert_close(y.float().cpu(), (x32 @ w32.t()).to(torch.bfloat16).float(), rtol=2e-2, atol=2e-2)
    dw_ref = (dy32.t() @ x32)
    scale = dw_ref.abs().max()
    assert float((w.grad.double().cpu() - dw_ref).abs().max() / scale) < 8e-3
    dx_ref = dy32 @ w32
    assert float((x.grad.double().cpu() - dx_ref).abs().max() / dx_ref.abs().max()) < 8e-3


@pytest.mark.gpu
def test_train_step_matches_torch_twin():
    cfg = gpt.GPTConfig(vocab_size=1024, d_model=256, n_layers=2, n_heads=4, head_dim=64,
                        d_ff=512, max_seq_len=256)
    tc = gpt.TrainConfig(batch=4, seq_len=256, lr=1e-3)
    res = gpt.parity(8, cfg, tc, torch.device("cuda"), learnable=True)
    for a, b in zip(res["loss_hip"], res["loss_torch"]):
        assert abs(a - b) / b < 0.01, (res["loss_hip"], res["loss_torch"])
    # the first step's gradients come from identical weights: their norms agree closely
    ga, gb = res["grad_norm_hip"][0], res["grad_norm_torch"][0]
    assert abs(ga - gb) / gb < 0.02, (ga, gb)
    # training moves the loss
    assert res["loss_hip"][-1] < res["loss_hip"][0]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("s,n", [(1, 8), (4, 768 * 768), (16, 2304 * 768), (3, 1001), (2, 6)])
def test_sum_splits_bitwise_against_ordered_fp32_sum(dtype, s, n):
    # tritium_sum_splits sums the split partials in fp32 in split order and rounds once:
    # bit-equal to the same ordered sum in torch (odd n takes the scalar path)
    g = torch.Generator().manual_seed(s * 1000 + n % 997)
    part = torch.randn((s, n), generator=g).cuda()
    want = part[0].clone()
    for j in range(1, s):
        want += part[j]
    got = gpt._sum_splits(part, dtype)
    assert torch.equal(got, want.to(dtype))
    # a misaligned source (offset by one element) takes the scalar path
    buf = torch.randn((s * n + 1,), generator=g).cuda()
    part2 = buf[1:].view(s, n)
    want2 = part2[0].clone()
    for j in range(1, s):
        want2 += part2[j]
    out = torch.empty(n, device="cuda", dtype=dtype)
    from helion_amd import _lib
    _lib.call("tritium_sum_splits", part2.data_ptr(), out.data_ptr(), s, n,
              _lib.dtype_code(dtype), _lib.stream_of(part2))
    assert torch.equal(out, want2.to(dtype))


@pytest.mark.gpu
def test_train_step_weight_gradients_on_second_stream_are_bitwise_equal():
    # HipGPT.train_step runs the projections' weight-gradient GEMMs on a second
    # stream (waited for before the update): the gradients and the updated
    # weights must be bitwise those of the one-stream step
    cfg = gpt.GPTConfig(vocab_size=1024, d_model=256, n_layers=2, n_heads=4, head_dim=64,
                        d_ff=512, max_seq_len=256)
    tc = gpt.TrainConfig(batch=4, seq_len=256, lr=1e-3)
    init = gpt.init_params(cfg, tc.seed)
    batch = gpt.lm_batch(cfg, tc, torch.Generator().manual_seed(3), torch.device("cuda"))
    out = {}
    saved = gpt.OVERLAP_DW
    try:
        for mode in (False, True):
            gpt.OVERLAP_DW = mode
            m = gpt.HipGPT(cfg, tc, init, torch.device("cuda"))
            losses = [float(m.train_step(*batch)) for _ in range(3)]
            out[mode] = (losses, [g.clone() for g in m._last_grads], m.master.flat.clone())
    finally:
        gpt.OVERLAP_DW = saved
    assert out[False][0] == out[True][0]
    assert all(torch.equal(a, b) for a, b in zip(out[False][1], out[True][1]))
    assert torch.equal(out[False][2], out[True][2])
