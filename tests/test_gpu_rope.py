"""RoPE on the GPU (mi_rope_apply / mi_rope_positions) against the CPU oracle.

Tolerance: the kernel and the oracle both compute the fp32 angle pos * f_i
and round the rotated value to the tensor dtype, so they differ by the output
rounding (half an ulp each side) plus what one fp32 ulp of f_i does at large
positions (pos * f_i * 2^-23 rad per ulp) times the pair's magnitude.
Dims past rotary_dim must come back bit-identical.
"""

import numpy as np
import pytest
import torch

from gpu_helpers import rope_bound
from oracle import rope as R

pytestmark = pytest.mark.gpu


def _check(x_in, x_out, pos, rd, interleave, scale, theta, llama31):
    ref = R.rope(x_in.cpu(), pos, rotary_dim=rd, interleave=interleave, rope_scale=scale, rope_theta=theta,
                 llama31=llama31)
    got = x_out.cpu().double()
    bound = rope_bound(x_in.cpu(), ref, pos, rd, interleave, scale, theta, llama31)
    err = (got - ref.double()).abs()
    assert (err <= bound).all(), f"max err {err.max().item():.3e}, worst ratio {(err / bound).max().item():.2f}"
    assert torch.equal(x_out[..., rd:].cpu(), x_in[..., rd:].cpu())


CASES = [
    # dtype, D, rotary_dim, interleave, scale, theta, llama31
    (torch.bfloat16, 128, 128, False, 1.0, 10000.0, None),
    (torch.bfloat16, 128, 64, False, 1.0, 1000000.0, None),
    (torch.float16, 64, 64, True, 2.0, 10000.0, None),
    (torch.bfloat16, 256, 256, True, 1.0, 10000.0, None),
    (torch.bfloat16, 128, 128, False, 8.0, 500000.0,
     dict(low_freq_factor=1.0, high_freq_factor=4.0, old_context_len=8192)),
    (torch.float16, 128, 96, False, 32.0, 500000.0,
     dict(low_freq_factor=1.0, high_freq_factor=4.0, old_context_len=8192)),
]


@pytest.mark.parametrize("dtype,d,rd,interleave,scale,theta,llama31", CASES)
@pytest.mark.parametrize("pos_dtype", [torch.int32, torch.int64])
def test_rope_matches_oracle(gpu, dtype, d, rd, interleave, scale, theta, llama31, pos_dtype):
    from mstar_amd import rope as MR

    g = torch.Generator().manual_seed(d * 7 + rd)
    t, hq, hkv = 37, 8, 2
    q = torch.randn(t, hq, d, generator=g).to(dtype)
    k = torch.randn(t, hkv, d, generator=g).to(dtype)
    pos = torch.cat([torch.arange(8), torch.randint(0, 32768, (t - 8,), generator=g)]).to(pos_dtype)
    qg, kg = q.to(gpu), k.to(gpu)
    if llama31:
        MR.apply_llama31_rope_pos_ids_inplace(qg, kg, pos.to(gpu), rotary_dim=rd, interleave=interleave,
                                              rope_scale=scale, rope_theta=theta, **llama31)
    else:
        MR.apply_rope_pos_ids_inplace(qg, kg, pos.to(gpu), rotary_dim=rd, interleave=interleave,
                                      rope_scale=scale, rope_theta=theta)
    torch.cuda.synchronize()
    _check(q, qg, pos.numpy(), rd, interleave, scale, theta, llama31)
    _check(k, kg, pos.numpy(), rd, interleave, scale, theta, llama31)


def test_rope_strided_views(gpu):
    """q and k as views of one fused projection output (token stride > heads * D)."""
    from mstar_amd import rope as MR

    t, hq, hkv, d = 19, 4, 2, 128
    qkv = torch.randn(t, (hq + 2 * hkv) * d, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    g = qkv.to(gpu)
    q = g[:, : hq * d].view(t, hq, d)
    k = g[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    pos = torch.arange(100, 100 + t, device=gpu)
    MR.apply_rope_pos_ids_inplace(q, k, pos)
    torch.cuda.synchronize()
    q0 = qkv[:, : hq * d].view(t, hq, d)
    k0 = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    _check(q0, q, pos.cpu().numpy(), d, False, 1.0, 1e4, None)
    _check(k0, k, pos.cpu().numpy(), d, False, 1.0, 1e4, None)
    assert torch.equal(g[:, (hq + hkv) * d:].cpu(), qkv[:, (hq + hkv) * d:])  # v untouched


def test_reference_rope_scenario(gpu):
    """test_flashinfer_rope_matches_hf_gemma_formula (test_pi05_reference_equivalence.py:592-617)."""
    from mstar_amd import rope as MR

    torch.manual_seed(0)
    seq_len, hq, hkv, d, theta = 8, 8, 1, 256, 10000.0
    q = torch.randn(seq_len, hq, d, dtype=torch.bfloat16)
    k = torch.randn(seq_len, hkv, d, dtype=torch.bfloat16)
    pos = torch.arange(seq_len, dtype=torch.int32)
    q_ref = R.rope(q, pos.numpy(), rope_theta=theta).to(torch.bfloat16)
    k_ref = R.rope(k, pos.numpy(), rope_theta=theta).to(torch.bfloat16)
    qg, kg = q.to(gpu), k.to(gpu)
    MR.apply_rope_pos_ids_inplace(qg, kg, pos.to(gpu), rope_theta=theta)
    assert (qg.cpu().float() - q_ref.float()).abs().max().item() < 1e-2
    assert (kg.cpu().float() - k_ref.float()).abs().max().item() < 1e-2


def test_manager_plan_and_apply_rope(gpu):
    """BatchedCacheManager.plan_rope/apply_rope: positions bit-exact, fp32 inputs rotated in bf16."""
    from mstar_amd.cache_manager import BatchedCacheManager, WorkspaceBufferManager
    from mstar_amd.kv_store import KVCacheConfig, PagedAllocationManager

    hq, hkv, d = 8, 2, 128
    cfg = KVCacheConfig(num_layers=1, num_kv_heads=hkv, head_dim=d, max_seq_len=4096, max_num_pages=256,
                        page_size=16, num_qo_heads=hq)
    kv = torch.zeros(1, 256, 2, 16, hkv, d, dtype=torch.bfloat16, device=gpu)
    mgr = PagedAllocationManager(cfg, kv, device=gpu)
    rids = ["a", "b", "c"]
    starts = [0, 1000, 77]
    for r, s0 in zip(rids, starts):
        mgr.add_request(r, ["main"])
        mgr.get_state(r, "main").position_id_start = s0
    cm = BatchedCacheManager(rids, {r: "main" for r in rids}, kv, mgr, WorkspaceBufferManager(64 << 20, gpu), cfg, gpu)
    seq_lens = [5, 1, 12]
    cm.plan_rope(seq_lens)
    pos = cm._plan_states["main"].pos_ids
    assert pos.dtype == torch.int64
    assert pos.cpu().numpy().tolist() == R.positions(seq_lens, starts).tolist()
    t = sum(seq_lens)
    q = torch.randn(t, hq, d, generator=torch.Generator().manual_seed(9))
    k = torch.randn(t, hkv, d, generator=torch.Generator().manual_seed(10))
    qo, ko = cm.apply_rope(q.to(gpu), k.to(gpu), rope_theta=500000.0)
    assert qo.dtype == torch.float32 and ko.dtype == torch.float32
    qb, kb = q.to(torch.bfloat16), k.to(torch.bfloat16)
    _check(qb, qo.to(torch.bfloat16), pos.cpu().numpy(), d, False, 1.0, 500000.0, None)
    _check(kb, ko.to(torch.bfloat16), pos.cpu().numpy(), d, False, 1.0, 500000.0, None)
    # explicit positions pass straight through
    cm.plan_rope(seq_lens, pos_ids=torch.arange(t, dtype=torch.int32))
    assert cm._plan_states["main"].pos_ids.cpu().tolist() == list(range(t))
