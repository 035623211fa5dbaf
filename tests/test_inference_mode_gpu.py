"""Blocks whose weights were made under torch.inference_mode (tensors with no
version counter) run forward and step, and give the same results as the same
weights made outside it: the derived weight copies (the transposed prefill
operand and the packed decode operand) are keyed by storage for such tensors."""

import dataclasses

import pytest

pytestmark = pytest.mark.gpu


def _inference_copy(m):
    import torch
    with torch.inference_mode():
        fields = {f.name: getattr(m, f.name) for f in dataclasses.fields(m) if f.init}
        return dataclasses.replace(m, **{k: v.clone() for k, v in fields.items() if isinstance(v, torch.Tensor)})


def test_mamba2_forward_inference_mode_weights():
    import torch
    import mamba_hip
    cfg = mamba_hip.Mamba2Config(d_model=64, state_rank=16, per_head_dim=16)
    m = cfg.init("cuda", torch.bfloat16, torch.Generator().manual_seed(3))
    mi = _inference_copy(m)
    x = torch.randn((2, 40, 64), generator=torch.Generator(device="cuda").manual_seed(4), device="cuda")
    with torch.inference_mode():
        got, _ = mi.forward(x.to(torch.bfloat16), None, chunk_len=16)
        got2, _ = mi.forward(x.to(torch.bfloat16), None, chunk_len=16)  # the cached copy is reused
    want, _ = m.forward(x.to(torch.bfloat16), None, chunk_len=16)
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(got2, want)


def test_mamba3_forward_and_step_inference_mode_weights():
    import torch
    import mamba_hip
    cfg = mamba_hip.Mamba3Config(d_model=128, state_rank=128, per_head_dim=64, mimo_rank=4)
    m = cfg.init("cuda", torch.bfloat16, torch.Generator(device="cuda").manual_seed(5))
    mi = _inference_copy(m)
    gen = torch.Generator(device="cuda").manual_seed(6)
    x = torch.randn((2, 50, 128), generator=gen, device="cuda").to(torch.bfloat16)
    xt = torch.randn((2, 128), generator=gen, device="cuda").to(torch.bfloat16)
    with torch.inference_mode():
        mi.pack_products()
        o1, c1 = mi.forward(x, None, chunk_len=32)
        s1, c1 = mi.step(xt, c1)
    o2, c2 = m.forward(x, None, chunk_len=32)
    s2, c2 = m.step(xt, c2)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    assert torch.equal(c1.ssm_bhpr, c2.ssm_bhpr)


def test_mamba3_inference_mode_weight_update_then_drop_derived():
    """An in-place update of an inference-mode in_proj weight, followed by
    drop_derived, reaches forward: the padded prefill copy (in_proj rows are
    padded to 8 elements, d_in_proj = 2 d_inner + ... is rarely a multiple of
    8) is forgotten with the others."""
    import torch
    import mamba_hip
    cfg = mamba_hip.Mamba3Config(d_model=128, state_rank=128, per_head_dim=64, mimo_rank=4)
    m = cfg.init("cuda", torch.bfloat16, torch.Generator(device="cuda").manual_seed(7))
    assert m.in_proj_w.shape[1] % 8 != 0  # the padded-copy case
    mi = _inference_copy(m)
    gen = torch.Generator(device="cuda").manual_seed(8)
    x = torch.randn((2, 40, 128), generator=gen, device="cuda").to(torch.bfloat16)
    delta = (0.05 * torch.randn(m.in_proj_w.shape, generator=gen, device="cuda")).to(torch.bfloat16)
    with torch.inference_mode():
        before, _ = mi.forward(x, None, chunk_len=32)
        mi.in_proj_w.add_(delta)
        mamba_hip.drop_derived(mi.in_proj_w)
        got, _ = mi.forward(x, None, chunk_len=32)
    fresh = dataclasses.replace(m, in_proj_w=(m.in_proj_w + delta).contiguous())
    want, _ = fresh.forward(x, None, chunk_len=32)
    torch.cuda.synchronize()
    assert not torch.equal(before, want)
    assert torch.equal(got, want)
