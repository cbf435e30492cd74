"""Write the golden fixtures of this directory from the CPU oracle.

The reference holds no stored vectors for this path (its tests compute
expected values on the fly), so these fixtures freeze the oracle's outputs on
small seeded inputs.  ``tests/test_golden.py`` checks that the oracle still
reproduces them exactly and that the GPU path matches them (bit-exact for
packing, page scatter and fp8 codes; the attention/RoPE tolerances for the
floating-point outputs; attention outputs are stored as fp16).

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import attention as A  # noqa: E402
from oracle import packing as P  # noqa: E402
from oracle import rope as R  # noqa: E402


def bf16_bits(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).view(torch.int16).numpy()


def packing() -> dict:
    """Two steps of FIFO allocation + packing: a prefill step, then a decode step."""
    ps, pool_n = 16, 48
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, 90, size=7)
    prompt[2] = 0  # a zero-length request (last_page_len = page_size quirk)
    pool = P.FifoPages(pool_n)
    states = [P.ReqState() for _ in prompt]
    s1 = P.pack(states, prompt.tolist(), pool, ps)
    t2p1, t2c1 = P.token_map(s1.qo_indptr, s1.kv_indptr, s1.kv_indices, s1.last_page_len, ps, tail_len=int(prompt.sum()) + 5)
    for st, n in zip(states, prompt):
        st.seq_len += int(n)
    pool.give(states[4].pages)  # request 4 finishes: its pages return to the tail of the free list
    states[4] = P.ReqState()
    s2 = P.pack(states, [1] * len(states), pool, ps)
    return dict(page_size=np.int32(ps), pool=np.int32(pool_n), prompt=prompt.astype(np.int32),
                qo1=s1.qo_indptr, kv1=s1.kv_indptr, idx1=s1.kv_indices, last1=s1.last_page_len,
                t2p1=t2p1, t2c1=t2c1, kv2=s2.kv_indptr, idx2=s2.kv_indices, last2=s2.last_page_len,
                loc2=s2.kv_locations, free_after=np.asarray(list(pool.free), dtype=np.int32))


def attention_case(qo_lens, kv_lens, hq, hkv, d, ps, pool_n, seed, causal) -> dict:
    g = torch.Generator().manual_seed(seed)
    cache = torch.randn(pool_n, 2, ps, hkv, d, generator=g).to(torch.bfloat16)
    kv_lens = np.asarray(kv_lens)
    npages = (kv_lens + ps - 1) // ps
    perm = torch.randperm(pool_n, generator=g).numpy().astype(np.int32)
    kv_indptr = np.concatenate([[0], np.cumsum(npages)]).astype(np.int32)
    qo = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    last = (kv_lens - (npages - 1) * ps).astype(np.int32)
    idx = perm[: kv_indptr[-1]]
    q = torch.randn(int(qo[-1]), hq, d, generator=g).to(torch.bfloat16)
    out = A.paged_attention(q, cache, qo, kv_indptr, idx, last, causal=causal)
    return dict(cache=bf16_bits(cache), q=bf16_bits(q), qo_indptr=qo, kv_indptr=kv_indptr, kv_indices=idx,
                last_page_len=last, out=out.numpy().astype(np.float16), causal=np.int32(causal),
                num_kv_heads=np.int32(hkv))


def rope_case() -> dict:
    g = torch.Generator().manual_seed(21)
    q = torch.randn(11, 4, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(11, 2, 128, generator=g).to(torch.bfloat16)
    pos = torch.cat([torch.arange(6), torch.tensor([100, 4095, 8192, 20000, 32767])]).numpy()
    l31 = dict(low_freq_factor=1.0, high_freq_factor=4.0, old_context_len=8192)
    return dict(q=bf16_bits(q), k=bf16_bits(k), pos=pos.astype(np.int64),
                q_plain=R.rope(q, pos, rope_theta=1e4).numpy(), k_plain=R.rope(k, pos, rope_theta=1e4).numpy(),
                q_l31=R.rope(q, pos, rope_scale=8.0, rope_theta=5e5, llama31=l31).numpy(),
                k_l31=R.rope(k, pos, rope_scale=8.0, rope_theta=5e5, llama31=l31).numpy())


def fp8_case() -> dict:
    g = torch.Generator().manual_seed(31)
    x = torch.randn(9, 2, 64, generator=g) * 3
    s = A.head_scales(x)
    x[0, 0, :4] = torch.tensor([1e6, -1e6, 0.0, -0.0])  # past +-448 after scaling: saturates; signed zeros
    return dict(x=x.numpy(), scale=s.numpy(), codes=A.quantize_e4m3(x, s).view(torch.uint8).numpy())


def main() -> None:
    np.savez_compressed(HERE / "packing.npz", **packing())
    np.savez_compressed(HERE / "decode_small.npz",
                        **attention_case([1] * 5, [1, 15, 16, 17, 200], 8, 2, 64, 16, 24, 41, False))
    np.savez_compressed(HERE / "prefill_small.npz",
                        **attention_case([40, 1, 9], [40, 70, 9 + 33], 8, 2, 128, 16, 12, 51, True))
    np.savez_compressed(HERE / "rope_small.npz", **rope_case())
    np.savez_compressed(HERE / "fp8_codes.npz", **fp8_case())
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main()
