"""CPU tests of the decode products' fragment order (vesta/prefill.py
frag_weights / frag_offset, the layout hip/prefill.hip pf_mgemm* reads and
pf_frag_put8 writes): every element lands where the documented lane rule
puts it, and a 16 x 16 x 32 matrix-core tile evaluated from the two
fragment arrays by that rule equals the plain product."""
import numpy as np
import torch

from vesta.prefill import frag_offset, frag_weights


def test_weight_fragments_place_every_element_by_the_lane_rule():
    rng = np.random.default_rng(0)
    W = torch.from_numpy(rng.standard_normal((2, 40, 64)).astype(np.float32))      # [L, N, K], N not a multiple of 16
    f = frag_weights(W)
    assert tuple(f.shape) == (2, 3, 2, 64, 8)
    for l in range(2):
        for n in range(48):
            for k in range(64):
                got = f[l, n // 16, k // 32, 16 * ((k % 32) // 8) + n % 16, k % 8].item()
                assert got == (W[l, n, k].item() if n < 40 else 0.0), (l, n, k)


def test_activation_offsets_cover_both_planes_once():
    M16, K = 32, 96
    seen = set()
    for plane in range(2):
        for m in range(M16):
            for k in range(K):
                seen.add(frag_offset(M16, K, plane, m, k))
    assert seen == set(range(2 * M16 * K))


def test_fragment_tiles_multiply_like_the_plain_product():
    """C[i, j] = sum over lanes-groups q and positions e of A-lane (16q + i)
    times B-lane (16q + j): the operand rule of v_mfma_f32_16x16x32_f16
    applied to the two fragment arrays gives A @ W^T for every tile pair."""
    rng = np.random.default_rng(1)
    M, N, K = 32, 48, 96
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = rng.standard_normal((N, K)).astype(np.float32)
    Af = np.zeros(2 * M * K, np.float32)
    for m in range(M):
        for k in range(K):
            Af[frag_offset(M, K, 0, m, k)] = A[m, k]
    Af = Af.reshape(2, M // 16, K // 32, 64, 8)
    Wf = frag_weights(torch.from_numpy(W)).numpy()                                  # [N/16, K/32, 64, 8]
    C = np.zeros((M, N), np.float64)
    for mt in range(M // 16):
        for nt in range(N // 16):
            for kt in range(K // 32):
                a, b = Af[0, mt, kt], Wf[nt, kt]                                    # [64 lanes, 8]
                for i in range(16):
                    for j in range(16):
                        C[16 * mt + i, 16 * nt + j] += sum(float(a[16 * q + i] @ b[16 * q + j]) for q in range(4))
    assert np.abs(C - A.astype(np.float64) @ W.T.astype(np.float64)).max() < 1e-3


def test_decode_attention_kernel_follows_the_block_count():
    """The layered decode pass reads each cache row in one pass (pf_attn1s)
    when it has at most ATTN_ONE_PASS_BLOCKS (row, head) blocks, in two
    (pf_attn1) with more."""
    from types import SimpleNamespace
    from vesta import prefill
    pick = lambda B, H: prefill.Prefill._attn1(SimpleNamespace(m=SimpleNamespace(B=B, H=H)))   # noqa: E731
    n = prefill.ATTN_ONE_PASS_BLOCKS
    assert pick(n // 16, 16) == 'pf_attn1s' and pick(n // 16 + 1, 16) == 'pf_attn1'
    assert pick(32, 12) == 'pf_attn1s' and pick(64, 25) == 'pf_attn1'
    assert {'pf_attn1', 'pf_attn1s', 'pf_mhead1', 'pf_mhead2', 'pf_mhead4'} <= set(prefill.KERNELS)
    src = prefill.prefill_source(448)
    for name in ('pf_attn1s', 'pf_mhead1', 'pf_mhead2', 'pf_mhead4'):
        assert f'void {name}(' in src or f'PF_MHEAD({name},' in src, name
