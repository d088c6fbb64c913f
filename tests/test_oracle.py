"""CPU tests that pin the oracle (no GPU).

Each oracle function is checked against something it does not itself
compute: closed forms of the recurrence, an independent algorithm (token
recurrence vs chunked UT form, forward substitution vs a library triangular
solve, F.conv1d vs a scalar loop), and structural invariants (varlen ==
per-sequence, split prefill == one prefill, slot permutation).  The golden
fixtures in tests/golden freeze the oracle's answers.
"""
import math
import os

import pytest
import torch
import torch.nn.functional as F
from safetensors.torch import load_file

from myvllm_amd.workloads import conv_decode_case, conv_prefill_case, cu_from_lengths, gdn_inputs, prefill_case
from oracle.conv import causal_conv1d_fn_ref, causal_conv1d_loop_ref, causal_conv1d_update_ref
from oracle.gdn import (chunk_gated_delta_rule_fla_ref, chunk_gated_delta_rule_ref, recurrent_gated_delta_rule_ref,
                        tril_inverse_ref)
from oracle.layer import gdn_gating_ref, l2norm_ref, rms_norm_gated_ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _inputs(T, Hk=2, Hv=4, K=32, V=32, seed=0, dtype=torch.float64):
    gen = torch.Generator().manual_seed(seed)
    q, k, v, g, beta = gdn_inputs(gen, T, Hk, Hv, K, V, dtype=torch.float64)
    return q.to(dtype), k.to(dtype), v.to(dtype), g.double(), beta.double()


# ---- token recurrence: closed forms ------------------------------------------------


def test_single_token_from_zero_state():
    """S0 = 0: S1 = beta k v^T, o = scale (q.k) beta v."""
    q, k, v, g, beta = _inputs(1, Hk=2, Hv=4)
    st = torch.zeros(1, 4, 32, 32, dtype=torch.float64)
    o = recurrent_gated_delta_rule_ref(q, k, v, g, beta, st, torch.tensor([0]))
    scale = 32 ** -0.5
    for h in range(4):
        kh = k[0, h // 2]
        qk = float(q[0, h // 2] @ kh)
        assert torch.allclose(o[0, h], scale * qk * beta[0, h] * v[0, h], atol=1e-14)
        assert torch.allclose(st[0, h], beta[0, h] * torch.outer(kh, v[0, h]), atol=1e-14)


def test_beta_one_no_decay_writes_value_exactly():
    """beta = 1, g = 0, |k| = 1: after the update k^T S = v for any S0."""
    q, k, v, g, beta = _inputs(1, Hk=1, Hv=1, K=16, V=8)
    st = torch.randn(1, 1, 16, 8, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    recurrent_gated_delta_rule_ref(q, k, v, torch.zeros_like(g), torch.ones_like(beta), st, torch.tensor([0]))
    assert torch.allclose(k[0, 0] @ st[0, 0], v[0, 0], atol=1e-13)


def test_beta_zero_is_pure_decay():
    q, k, v, g, beta = _inputs(1, Hk=1, Hv=2, K=16, V=8)
    st0 = torch.randn(1, 2, 16, 8, dtype=torch.float64, generator=torch.Generator().manual_seed(2))
    st = st0.clone()
    o = recurrent_gated_delta_rule_ref(q, k, v, g, torch.zeros_like(beta), st, torch.tensor([0]))
    for h in range(2):
        dec = math.exp(float(g[0, h]))
        assert torch.allclose(st[0, h], dec * st0[0, h], atol=1e-14)
        assert torch.allclose(o[0, h], dec * (st0[0, h].t() @ q[0, 0]) * 16 ** -0.5, atol=1e-13)


def test_large_negative_decay_resets_state():
    q, k, v, g, beta = _inputs(1, Hk=1, Hv=1, K=16, V=8)
    st = torch.randn(1, 1, 16, 8, dtype=torch.float64, generator=torch.Generator().manual_seed(3)) * 100
    recurrent_gated_delta_rule_ref(q, k, v, torch.full_like(g, -1e4), beta, st, torch.tensor([0]))
    assert torch.allclose(st[0, 0], beta[0, 0] * torch.outer(k[0, 0], v[0, 0]), atol=1e-13)


def test_gva_head_map_is_h_div_r():
    """v-head h reads k-head h // (Hv / Hk): zero k-head 1 and only v-heads 2, 3 keep a pure-decay state."""
    q, k, v, g, beta = _inputs(3, Hk=2, Hv=4, K=16, V=8)
    k[:, 1] = 0
    st0 = torch.randn(1, 4, 16, 8, dtype=torch.float64, generator=torch.Generator().manual_seed(4))
    st = st0.clone()
    recurrent_gated_delta_rule_ref(q, k, v, g, beta, st, torch.tensor([0]), cu_seqlens=torch.tensor([0, 3]))
    for h in range(4):
        pure = st0[0, h] * math.exp(float(g[:, h].sum()))
        assert torch.allclose(st[0, h], pure, atol=1e-13) == (h // 2 == 1)


def test_padding_slot_is_skipped():
    q, k, v, g, beta = _inputs(2, Hk=1, Hv=1, K=8, V=8)
    st0 = torch.randn(2, 1, 8, 8, dtype=torch.float64)
    st = st0.clone()
    o = recurrent_gated_delta_rule_ref(q, k, v, g, beta, st, torch.tensor([-1, 1]))
    assert torch.count_nonzero(o[0]) == 0
    assert torch.equal(st[0], st0[0]) and not torch.equal(st[1], st0[1])


# ---- chunked form vs token recurrence ------------------------------------------------


@pytest.mark.parametrize("chunk", [16, 32, 64])
def test_chunked_equals_recurrence_fp64(chunk):
    lengths = [0, 5, 64, 70, 1, 129]
    cu = cu_from_lengths(lengths)
    T = int(cu[-1])
    q, k, v, g, beta = _inputs(T, Hk=2, Hv=4)
    st0 = 0.1 * torch.randn(9, 4, 32, 32, dtype=torch.float64, generator=torch.Generator().manual_seed(5))
    idx = torch.tensor([3, 0, 8, 5, 1, 2], dtype=torch.int32)
    s1, s2 = st0.clone(), st0.clone()
    o1 = recurrent_gated_delta_rule_ref(q, k, v, g, beta, s1, idx, cu)
    o2 = chunk_gated_delta_rule_ref(q, k, v, g, beta, s2, idx, cu, chunk_size=chunk)
    assert (o1 - o2).abs().max() < 1e-12
    assert (s1 - s2).abs().max() < 1e-12
    assert torch.equal(s2[[4, 6, 7]], st0[[4, 6, 7]])  # untouched slots


def test_triangular_inverse_matches_library():
    gen = torch.Generator().manual_seed(6)
    A = torch.tril(torch.randn(3, 64, 64, dtype=torch.float64, generator=gen) * 0.1, diagonal=-1)
    eye = torch.eye(64, dtype=torch.float64).expand_as(A)
    ref = torch.linalg.solve_triangular(eye + A, eye, upper=False)
    assert (tril_inverse_ref(A) - ref).abs().max() < 1e-12
    assert ((eye + A) @ tril_inverse_ref(A) - eye).abs().max() < 1e-12


def test_chunked_substitution_and_library_solve_agree():
    cu = cu_from_lengths([100, 30])
    q, k, v, g, beta = _inputs(130, Hk=1, Hv=2)
    st0 = 0.1 * torch.randn(2, 2, 32, 32, dtype=torch.float64)
    s1, s2 = st0.clone(), st0.clone()
    o1 = chunk_gated_delta_rule_ref(q, k, v, g, beta, s1, torch.tensor([0, 1]), cu, use_library_solve=True)
    o2 = chunk_gated_delta_rule_ref(q, k, v, g, beta, s2, torch.tensor([0, 1]), cu, use_library_solve=False)
    assert (o1 - o2).abs().max() < 1e-12 and (s1 - s2).abs().max() < 1e-12


def test_varlen_equals_per_sequence():
    lengths = [7, 65, 30]
    cu = cu_from_lengths(lengths)
    q, k, v, g, beta = _inputs(int(cu[-1]), Hk=2, Hv=4)
    st0 = 0.1 * torch.randn(3, 4, 32, 32, dtype=torch.float64)
    idx = torch.tensor([2, 0, 1])
    st = st0.clone()
    o = chunk_gated_delta_rule_ref(q, k, v, g, beta, st, idx, cu)
    for n in range(3):
        s, e = int(cu[n]), int(cu[n + 1])
        stn = st0[idx[n]: idx[n] + 1].clone()
        on = chunk_gated_delta_rule_ref(q[s:e], k[s:e], v[s:e], g[s:e], beta[s:e], stn, torch.tensor([0]),
                                        torch.tensor([0, e - s]))
        assert torch.equal(o[s:e], on)
        assert torch.equal(st[idx[n]], stn[0])


def test_split_prefill_equals_one_prefill():
    q, k, v, g, beta = _inputs(150, Hk=1, Hv=2)
    st0 = 0.1 * torch.randn(1, 2, 32, 32, dtype=torch.float64)
    a, b = st0.clone(), st0.clone()
    o_all = chunk_gated_delta_rule_ref(q, k, v, g, beta, a, torch.tensor([0]), torch.tensor([0, 150]))
    o1 = chunk_gated_delta_rule_ref(q[:90], k[:90], v[:90], g[:90], beta[:90], b, torch.tensor([0]),
                                    torch.tensor([0, 90]))
    o2 = chunk_gated_delta_rule_ref(q[90:], k[90:], v[90:], g[90:], beta[90:], b, torch.tensor([0]),
                                    torch.tensor([0, 60]))
    assert (torch.cat([o1, o2]) - o_all).abs().max() < 1e-12
    assert (a - b).abs().max() < 1e-12


def test_slot_permutation_permutes_results():
    cu = cu_from_lengths([20, 40])
    q, k, v, g, beta = _inputs(60, Hk=1, Hv=1)
    st0 = 0.1 * torch.randn(4, 1, 32, 32, dtype=torch.float64)
    a, b = st0.clone(), st0.clone()
    b[[1, 3]] = st0[[3, 1]]  # the same initial states, stored in swapped slots
    oa = chunk_gated_delta_rule_ref(q, k, v, g, beta, a, torch.tensor([1, 3]), cu)
    ob = chunk_gated_delta_rule_ref(q, k, v, g, beta, b, torch.tensor([3, 1]), cu)
    assert torch.equal(oa, ob)
    assert torch.equal(a[1], b[3]) and torch.equal(a[3], b[1])
    assert torch.equal(a[[0, 2]], st0[[0, 2]])


def test_decode_continues_prefill():
    """Prefill of L tokens then one recurrent step == recurrence over L + 1 tokens."""
    q, k, v, g, beta = _inputs(41, Hk=1, Hv=2)
    st0 = 0.1 * torch.randn(1, 2, 32, 32, dtype=torch.float64)
    a, b = st0.clone(), st0.clone()
    chunk_gated_delta_rule_ref(q[:40], k[:40], v[:40], g[:40], beta[:40], a, torch.tensor([0]), torch.tensor([0, 40]))
    o_dec = recurrent_gated_delta_rule_ref(q[40:], k[40:], v[40:], g[40:], beta[40:], a, torch.tensor([0]))
    o_all = recurrent_gated_delta_rule_ref(q, k, v, g, beta, b, torch.tensor([0]), torch.tensor([0, 41]))
    assert (o_dec[0] - o_all[40]).abs().max() < 1e-12 and (a - b).abs().max() < 1e-12


def test_functional_form_matches_cache_form():
    cu = cu_from_lengths([33, 12])
    q, k, v, g, beta = _inputs(45, Hk=1, Hv=2)
    init = 0.1 * torch.randn(2, 2, 32, 32, dtype=torch.float64)
    o, fin = chunk_gated_delta_rule_fla_ref(q, k, v, g, beta, cu, initial_state=init, output_final_state=True)
    st = init.clone()
    o2 = chunk_gated_delta_rule_ref(q, k, v, g, beta, st, torch.tensor([0, 1]), cu)
    assert torch.equal(o, o2) and torch.equal(fin, st)


# ---- conv -----------------------------------------------------------------------------


@pytest.mark.parametrize("W", [2, 4, 6])
def test_conv_matches_scalar_loop(W):
    c = conv_prefill_case([3, 1, 9, 0, 2], seed=W, D=8, W=W, num_slots=6, dtype=torch.float32)
    st = c.state.clone()
    y = causal_conv1d_fn_ref(c.x, c.weight, st, c.idx, c.cu)
    y2, st2 = causal_conv1d_loop_ref(c.x, c.weight, c.state, c.idx, c.cu)
    assert (y.double() - y2).abs().max() < 1e-6  # y is returned in x's dtype (fp32)
    assert torch.allclose(st.double(), st2.double(), atol=0, rtol=0)


def test_conv_new_state_is_last_rows_and_short_sequences_keep_old_rows():
    c = conv_prefill_case([1, 5], seed=1, D=16, W=4, num_slots=2, dtype=torch.float32)
    st = c.state.clone()
    causal_conv1d_fn_ref(c.x, c.weight, st, c.idx, c.cu)
    s0, s1 = int(c.idx[0]), int(c.idx[1])
    assert torch.equal(st[s0], torch.cat([c.state[s0][1:], c.x[0:1]]))  # 1 token: shift by one
    assert torch.equal(st[s1], c.x[3:6])


def test_conv_update_equals_one_token_prefill():
    c = conv_decode_case(B=4, seed=2, D=16, W=4, num_slots=6, dtype=torch.float32)
    a, b = c.state.clone(), c.state.clone()
    ya = causal_conv1d_update_ref(c.x, c.weight, a, c.idx)
    yb = causal_conv1d_fn_ref(c.x, c.weight, b, c.idx, cu_from_lengths([1] * 4))
    assert torch.equal(ya, yb) and torch.equal(a, b)


def test_conv_equals_torch_conv1d_with_zero_state():
    """With a zero initial state the prefill is F.conv1d with causal left padding."""
    c = conv_prefill_case([12], seed=3, D=8, W=4, num_slots=1, dtype=torch.float32)
    st = torch.zeros_like(c.state)
    y = causal_conv1d_fn_ref(c.x, c.weight, st, c.idx, c.cu)
    ref = F.silu(F.conv1d(F.pad(c.x.double().t()[None], (3, 0)), c.weight.double()[:, None, :], groups=8))[0].t()
    assert (y.double() - ref).abs().max() < 1e-6


# ---- layer glue -----------------------------------------------------------------------


def test_gating_closed_forms():
    a = torch.zeros(1, 2)
    b = torch.zeros(1, 2)
    g, beta = gdn_gating_ref(a, b, torch.log(torch.tensor([1.0, 4.0])), torch.zeros(2))
    assert torch.allclose(beta, torch.full((1, 2), 0.5))
    assert torch.allclose(g, -torch.tensor([[1.0, 4.0]]) * math.log(2.0))


def test_l2norm_and_gated_rmsnorm_closed_forms():
    x = torch.tensor([[3.0, 4.0]])
    assert torch.allclose(l2norm_ref(x, eps=0.0), torch.tensor([[0.6, 0.8]]))
    gate = torch.zeros(1, 2)  # silu(0) = 0
    assert torch.count_nonzero(rms_norm_gated_ref(x, gate, torch.ones(2))) == 0
    gate = torch.full((1, 2), 50.0)  # silu(50) == 50 in fp32
    y = rms_norm_gated_ref(x, gate, torch.ones(2), eps=0.0)
    assert torch.allclose(y, x / math.sqrt(12.5) * 50.0)


# ---- golden fixtures ------------------------------------------------------------------


def test_golden_recurrent_64tok():
    f = load_file(os.path.join(GOLDEN, "gdn_recurrent_64tok.safetensors"))
    st = torch.zeros(1, 32, 128, 128)
    o = recurrent_gated_delta_rule_ref(f["q"], f["k"], f["v"], f["g"], f["beta"], st, f["state_indices"],
                                       f["cu_seqlens"])
    assert (o - f["o"]).abs().max() < 1e-6
    assert (st[0] - f["final_state"]).abs().max() < 1e-6
    # the chunked form reproduces it too
    st2 = torch.zeros(1, 32, 128, 128)
    o2 = chunk_gated_delta_rule_ref(f["q"], f["k"], f["v"], f["g"], f["beta"], st2, f["state_indices"],
                                    f["cu_seqlens"])
    assert (o2 - f["o"]).abs().max() < 1e-5 and (st2[0] - f["final_state"]).abs().max() < 1e-5


def test_golden_chunk_varlen_small():
    f = load_file(os.path.join(GOLDEN, "gdn_chunk_varlen_small.safetensors"))
    st = f["initial_state"].clone()
    o = chunk_gated_delta_rule_ref(f["q"], f["k"], f["v"], f["g"], f["beta"], st, f["state_indices"],
                                   f["cu_seqlens"], dtype=torch.float64)
    assert (o.float() - f["o"]).abs().max() < 2e-2  # o is stored in the inputs' bf16
    assert (st - f["final_state"]).abs().max() < 1e-6


def test_golden_decode_small():
    f = load_file(os.path.join(GOLDEN, "gdn_decode_small.safetensors"))
    st = f["initial_state"].clone()
    o = recurrent_gated_delta_rule_ref(f["q"], f["k"], f["v"], f["g"], f["beta"], st, f["state_indices"])
    assert (o.float() - f["o"]).abs().max() < 1e-2
    assert (st - f["final_state"]).abs().max() < 1e-6


def test_golden_conv():
    f = load_file(os.path.join(GOLDEN, "conv_varlen_small.safetensors"))
    st = f["initial_state"].clone()
    y = causal_conv1d_fn_ref(f["x"], f["weight"], st, f["state_indices"], f["cu_seqlens"])
    assert (y.float() - f["y"]).abs().max() < 1e-3 and torch.equal(st, f["final_state"])
    f = load_file(os.path.join(GOLDEN, "conv_update_small.safetensors"))
    st = f["initial_state"].clone()
    y = causal_conv1d_update_ref(f["x"], f["weight"], st, f["state_indices"])
    assert (y.float() - f["y"]).abs().max() < 1e-3 and torch.equal(st, f["final_state"])


def test_golden_attention():
    from oracle.attention import flash_attention_prefill_ref, paged_attention_ref
    from myvllm_amd.workloads import cu_from_lengths

    f = load_file(os.path.join(GOLDEN, "attn_varlen_small.safetensors"))
    o = flash_attention_prefill_ref(f["q"], f["k"], f["v"], f["cu_seqlens"], float(f["scale"]), is_causal=True)
    assert (o.float() - f["o"]).abs().max() < 1e-6
    f = load_file(os.path.join(GOLDEN, "attn_paged_small.safetensors"))
    o = paged_attention_ref(f["q"], f["k_cache"], f["v_cache"], f["block_tables"], f["context_lens"],
                            f["cu_seqlens"], float(f["scale"]))
    assert (o.float() - f["o"]).abs().max() < 1e-6
    od = paged_attention_ref(f["decode_q"], f["k_cache"], f["v_cache"], f["block_tables"], f["decode_context_lens"],
                             cu_from_lengths([1, 1, 1]), float(f["scale"]))
    assert (od.float() - f["decode_o"]).abs().max() < 1e-6


def test_workload_lengths_match_the_benchmark_description():
    from myvllm_amd.workloads import conv_prefill_case as cp, prefill_32k_case

    assert cp().cu.diff().tolist() == [2943, 3503, 2192, 1807, 3696, 649, 3521, 1451]
    c = prefill_32k_case()
    assert c.tokens == 35846 and int(((c.cu.diff() + 63) // 64).sum()) == 567


# ---- full-attention neighbour -------------------------------------------------------

from oracle.attention import attention_loop_ref, flash_attention_prefill_ref, paged_attention_ref  # noqa: E402


def test_attention_matches_scalar_loops_with_gqa():
    g = torch.Generator().manual_seed(11)
    q, k, v = torch.randn(5, 4, 3, generator=g), torch.randn(5, 2, 3, generator=g), torch.randn(5, 2, 2, generator=g)
    for causal in (True, False):
        o = flash_attention_prefill_ref(q, k, v, torch.tensor([0, 5]), 0.7, is_causal=causal)
        assert torch.allclose(o.double(), attention_loop_ref(q, k, v, 0.7, torch.arange(5), causal), atol=1e-6)


def test_attention_closed_forms():
    g = torch.Generator().manual_seed(12)
    v = torch.randn(6, 1, 4, generator=g, dtype=torch.float64)
    q = torch.randn(6, 2, 8, generator=g, dtype=torch.float64)
    k = torch.zeros(6, 1, 8, dtype=torch.float64)  # all scores equal: causal o_i = mean(v_0..v_i)
    o = flash_attention_prefill_ref(q, k, v, torch.tensor([0, 6]), 1.0, is_causal=True)
    means = torch.cumsum(v[:, 0], 0) / torch.arange(1, 7, dtype=torch.float64)[:, None]
    assert torch.allclose(o[:, 0], means) and torch.allclose(o[:, 1], means)
    assert torch.allclose(o[0, :, :], v[0, 0].expand(2, 4))  # the first token attends only to itself


def test_paged_attention_equals_contiguous_and_permuted_pages():
    g = torch.Generator().manual_seed(13)
    bs, L, n = 4, 11, 3  # 11 cached keys, the last 3 are this prefill's queries
    k = torch.randn(L, 2, 8, generator=g, dtype=torch.float64)
    v = torch.randn(L, 2, 8, generator=g, dtype=torch.float64)
    q = torch.randn(n, 4, 8, generator=g, dtype=torch.float64)
    table = torch.tensor([5, 1, 3])  # pages in any order
    kc = torch.zeros(6, bs, 2, 8, dtype=torch.float64)
    vc = torch.zeros(6, bs, 2, 8, dtype=torch.float64)
    for j in range(L):
        kc[table[j // bs], j % bs] = k[j]
        vc[table[j // bs], j % bs] = v[j]
    o = paged_attention_ref(q, kc, vc, table[None], torch.tensor([L]), torch.tensor([0, n]), 0.5)
    ref = attention_loop_ref(q, k, v, 0.5, torch.arange(L - n, L), True)
    assert torch.allclose(o, ref, atol=1e-9)
