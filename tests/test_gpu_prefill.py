"""GPU parity: fused chunked prefill vs the CPU oracle (chunked UT form in fp64)."""
import pytest
import torch

from conftest import assert_out_close, assert_state_close
from myvllm_amd import chunk_gated_delta_rule, chunk_gated_delta_rule_fwd, recurrent_gated_delta_rule
from myvllm_amd.gated_delta_rule import chunk_prefill_ex
from myvllm_amd.workloads import cu_from_lengths, prefill_32k_case, prefill_case
from oracle.gdn import chunk_gated_delta_rule_ref, recurrent_gated_delta_rule_ref

pytestmark = pytest.mark.gpu


def _run(case, dev, idx=None, cu=None, beta=None, items_per_wg=None, spin_limit=None):
    """The op on the GPU and the oracle on the CPU.  With items_per_wg or
    spin_limit the call goes through gdn_chunk_prefill_ex with that schedule
    (-1: the launcher's choice) and wait bound (-1: the default)."""
    idx = case.idx if idx is None else idx
    cu = case.cu if cu is None else cu
    beta = case.beta if beta is None else beta
    st_ref = case.state.clone()
    o_ref = chunk_gated_delta_rule_ref(case.q, case.k, case.v, case.g, beta, st_ref, idx, cu)
    st = case.state.to(dev)
    args = (case.q.to(dev), case.k.to(dev), case.v.to(dev), case.g.to(dev), beta.to(dev), st, idx.to(dev), cu.to(dev))
    if items_per_wg is None and spin_limit is None:
        o = chunk_gated_delta_rule(*args)
    else:
        o = torch.full(case.v.shape, float("nan"), dtype=case.v.dtype, device=dev)
        chunk_prefill_ex(*args, o, case.q.shape[-1] ** -0.5,
                         items_per_wg=-1 if items_per_wg is None else items_per_wg,
                         spin_limit=-1 if spin_limit is None else spin_limit)
    torch.cuda.synchronize()
    return o.cpu(), st.cpu(), o_ref, st_ref


def _check(case, o, st, o_ref, st_ref, idx=None):
    idx = case.idx if idx is None else idx
    assert_out_close(o, o_ref)
    sel = torch.tensor([int(i) for i in idx.tolist() if 0 <= int(i) < st.shape[0]], dtype=torch.long)
    assert_state_close(st[sel], st_ref[sel])
    untouched = torch.ones(st.shape[0], dtype=torch.bool)
    untouched[sel] = False
    assert torch.equal(st[untouched], case.state[untouched])


@pytest.mark.parametrize("lengths", [[64], [1], [5, 64, 65], [130, 0, 200, 3, 127, 128, 129]])
def test_prefill_varlen_edges(dev, lengths):
    case = prefill_case(lengths, seed=len(lengths), num_slots=len(lengths) + 3, Hk=2, Hv=4)
    o, st, o_ref, st_ref = _run(case, dev)
    _check(case, o, st, o_ref, st_ref)


@pytest.mark.parametrize("K, V", [(64, 64), (128, 64), (64, 128), (96, 32), (8, 120)])
def test_prefill_head_dims(dev, K, V):
    """Head dims below 128 (multiples of 8) run zero-padded to 128: keys past K
    and values past V stay zero in the tiles and the state, the rest is exact."""
    case = prefill_case([200, 1, 65, 130], seed=K + V, num_slots=6, Hk=2, Hv=4, K=K, V=V)
    print(f"prefill head dims K={K} V={V}", flush=True)
    o, st, o_ref, st_ref = _run(case, dev)
    _check(case, o, st, o_ref, st_ref)


def test_prefill_head_dim_64_item_stream_fp16(dev):
    """d 64, fp16 q/k/v, 600 short sequences: the several-items-per-workgroup
    schedule with zero-padded head dims."""
    g = torch.Generator().manual_seed(21)
    lengths = torch.randint(1, 100, (600,), generator=g).tolist()
    case = prefill_case(lengths, seed=22, num_slots=640, Hk=1, Hv=2, K=64, V=64, dtype=torch.float16)
    print(f"prefill d64 fp16 item stream T={int(case.cu[-1])}", flush=True)
    o, st, o_ref, st_ref = _run(case, dev)
    _check(case, o, st, o_ref, st_ref)


def test_prefill_gva_ratio_one_and_four(dev):
    for Hk, Hv in ((4, 4), (1, 4)):
        case = prefill_case([70, 33], seed=7, num_slots=4, Hk=Hk, Hv=Hv)
        o, st, o_ref, st_ref = _run(case, dev)
        _check(case, o, st, o_ref, st_ref)


def test_prefill_weak_decay(dev):
    """g scaled by 0.01: the state carries across chunks, stressing the split-bf16 products."""
    case = prefill_case([300, 1000], seed=8, num_slots=2, Hk=2, Hv=4, g_scale=0.01)
    o, st, o_ref, st_ref = _run(case, dev)
    _check(case, o, st, o_ref, st_ref)


@pytest.mark.parametrize("state_scale", ["zero", "tiny", "large", "mixed"])
def test_prefill_initial_state_magnitudes(dev, state_scale):
    """Zero, tiny (1e-20), large (1e6) and per-value-column mixed (1e-15 .. 1e15)
    initial states under weak decay: the kernel holds the state in power-of-two
    units per value column, which must follow it from any starting magnitude.
    Outputs and states are compared in units of their value column's state
    scale where it exceeds 1: the bars' absolute floors are stated for
    unit-scale data (at 1e6 one bf16 ulp is ~4e3 and one fp32 ulp ~0.06)."""
    case = prefill_case([200, 70], seed=13, num_slots=3, Hk=2, Hv=4, g_scale=0.05)
    col = torch.ones(case.state.shape[-1], dtype=torch.float64)
    if state_scale == "zero":
        case.state.zero_()
    elif state_scale == "tiny":
        case.state.mul_(1e-19)
    elif state_scale == "large":
        case.state.mul_(1e7)
        col.fill_(1e7)
    else:
        col = torch.logspace(-15, 15, case.state.shape[-1], dtype=torch.float64)
        case.state.mul_(col.float())
    o, st, o_ref, st_ref = _run(case, dev)
    unit = col.clamp_min(1.0)
    assert_out_close(o.double() / unit, o_ref.double() / unit)
    sel = case.idx.long()
    assert_state_close(st[sel].double() / unit, st_ref[sel].double() / unit)


@pytest.mark.parametrize("g_scale", [1.6, 4.0])
def test_prefill_strong_decay(dev, g_scale):
    """Log-decays scaled up so that a chunk's cumulative decay passes e^-80
    (some chunks at 1.6, all at 4): the decay factors then take one exponential
    per entry instead of the product of per-token exponentials."""
    case = prefill_case([400, 130, 64], seed=14, num_slots=3, Hk=2, Hv=4, g_scale=g_scale)
    o, st, o_ref, st_ref = _run(case, dev)
    _check(case, o, st, o_ref, st_ref)


def test_prefill_long_no_decay(dev):
    """4,096 tokens (64 chunks) with g = 0: the state never decays, so its
    per-column units and magnitude bound are carried through every chunk."""
    case = prefill_case([4096], seed=15, num_slots=1, Hk=1, Hv=2)
    case.g.zero_()
    o, st, o_ref, st_ref = _run(case, dev)
    _check(case, o, st, o_ref, st_ref)


def test_prefill_zero_decay_beta_one(dev):
    """g = 0, beta = 1: pure delta rule, no decay at all."""
    case = prefill_case([256], seed=9, num_slots=1, Hk=1, Hv=2)
    case.g.zero_()
    case.beta.fill_(1.0)
    o, st, o_ref, st_ref = _run(case, dev)
    _check(case, o, st, o_ref, st_ref)


def test_prefill_padding_slot_int64_bf16_beta(dev):
    case = prefill_case([40, 90, 17], seed=10, num_slots=5, Hk=2, Hv=4, beta_dtype=torch.bfloat16)
    idx = case.idx.long().clone()
    idx[1] = -1
    o, st, o_ref, st_ref = _run(case, dev, idx=idx, cu=case.cu.long())
    assert torch.count_nonzero(o[40:130]) == 0
    _check(case, o, st, o_ref, st_ref, idx=idx)


def test_prefill_split_equals_whole_and_decode_continues(dev):
    """Prefill of 150 tokens == prefill 100 then 50 (carried state) == prefill 149 then one decode step."""
    case = prefill_case([150], seed=11, num_slots=1, Hk=2, Hv=4)
    q, k, v, g, b = (t.to(dev) for t in (case.q, case.k, case.v, case.g, case.beta))
    idx = case.idx.to(dev)
    st_a = case.state.to(dev)
    o_a = chunk_gated_delta_rule(q, k, v, g, b, st_a, idx, cu_from_lengths([150]).to(dev))
    st_b = case.state.to(dev)
    o_b1 = chunk_gated_delta_rule(q[:100], k[:100], v[:100], g[:100], b[:100], st_b, idx, cu_from_lengths([100]).to(dev))
    o_b2 = chunk_gated_delta_rule(q[100:], k[100:], v[100:], g[100:], b[100:], st_b, idx, cu_from_lengths([50]).to(dev))
    st_c = case.state.to(dev)
    o_c1 = chunk_gated_delta_rule(q[:149], k[:149], v[:149], g[:149], b[:149], st_c, idx, cu_from_lengths([149]).to(dev))
    o_c2 = recurrent_gated_delta_rule(q[149:], k[149:], v[149:], g[149:], b[149:], st_c, idx)
    assert_out_close(torch.cat([o_b1, o_b2]), o_a.float())
    assert_out_close(torch.cat([o_c1, o_c2]), o_a.float())
    assert_state_close(st_b, st_a)
    assert_state_close(st_c, st_a)


def test_prefill_functional_form(dev):
    case = prefill_case([77, 10], seed=12, num_slots=2, Hk=2, Hv=4)
    init = case.state[case.idx.long()]
    o, fin = chunk_gated_delta_rule_fwd(
        case.q.to(dev), case.k.to(dev), case.v.to(dev), case.g.to(dev), case.beta.to(dev), case.cu.to(dev),
        initial_state=init.to(dev), output_final_state=True,
    )
    st_ref = init.clone()
    o_ref = chunk_gated_delta_rule_ref(case.q, case.k, case.v, case.g, case.beta, st_ref,
                                       torch.arange(2, dtype=torch.int32), case.cu)
    assert_out_close(o, o_ref)
    assert_state_close(fin, st_ref)


def test_prefill_32k_full(dev):
    """Benchmark shape: 16 sequences, 35,846 tokens, Hk 16 / Hv 32, d 128, fp32 initial state."""
    case = prefill_32k_case()
    assert case.tokens == 35846
    o, st, o_ref, st_ref = _run(case, dev)
    _check(case, o, st, o_ref, st_ref)


@pytest.mark.parametrize("key", ["norm1", "norm8", "norm64", "norm128", "spiky8", "spiky128"])
def test_prefill_key_magnitudes(dev, key):
    """Keys that are not unit vectors: L2 norms 1, 8, 64 and 128 (the largest
    the C ABI accepts) in random directions, and norm-8 and norm-128 keys whose
    mass sits in one coordinate (|k_i| near 8 and 128), under weak decay over
    many chunks.  beta is divided by |k|^2 so the
    delta rule stays contractive (1 - beta |k|^2 in (0, 1)), as the unit-key
    recurrence is.  The state then scales like 1 / |k|, so outputs and states
    are compared after multiplying by |k| (the bars are stated for unit-scale
    data).  The state-update split is sized from each chunk's largest key
    norm; before that it assumed |k| <= 1."""
    case = prefill_case([700, 300, 64], seed=21, num_slots=4, Hk=2, Hv=4, g_scale=0.05)
    gen = torch.Generator().manual_seed(22)
    k = torch.nn.functional.normalize(torch.randn(case.k.shape, generator=gen), dim=-1)
    if key.startswith("spiky"):
        rho = float(key[5:])
        k = k * 0.05
        hot = torch.randint(0, k.shape[-1], k.shape[:2], generator=gen)
        k.scatter_(-1, hot[..., None], 1.0)
        k = torch.nn.functional.normalize(k, dim=-1)
    else:
        rho = float(key[4:])
    case.k = (k * rho).to(torch.bfloat16)
    case.beta = case.beta / case.k.float().pow(2).sum(-1).amax().item()
    case.state.mul_(1.0 / rho)
    print(f"prefill keys {key}: max |k| entry {case.k.float().abs().max().item():.2f}", flush=True)
    o, st, o_ref, st_ref = _run(case, dev)
    assert_out_close(o.double() * rho, o_ref.double() * rho)
    sel = case.idx.long()
    assert_state_close(st[sel].double() * rho, st_ref[sel].double() * rho)
    untouched = torch.ones(st.shape[0], dtype=torch.bool)
    untouched[sel] = False
    assert torch.equal(st[untouched], case.state[untouched])


def test_prefill_more_than_256_sequences(dev):
    """300 sequences of 0..200 tokens (a chunked-prefill scheduler's batch):
    past 256 sequences the kernel takes them in index order instead of
    longest first."""
    gen = torch.Generator().manual_seed(23)
    lengths = torch.randint(0, 201, (300,), generator=gen).tolist()
    lengths[7] = 0
    case = prefill_case(lengths, seed=24, num_slots=320, Hk=2, Hv=4)
    print(f"prefill 300 sequences, {case.tokens} tokens", flush=True)
    o, st, o_ref, st_ref = _run(case, dev)
    _check(case, o, st, o_ref, st_ref)


@pytest.mark.parametrize("lengths,g_scale", [([5, 64, 65, 200], 1.0), ([300, 1000], 0.01)])
def test_prefill_fp16(dev, lengths, g_scale):
    """fp16 q/k/v (the reference's prefill follows the inputs' dtype,
    ops/gated_delta_rule/wu.py:150-151, o.py:147): o comes back in fp16, the
    state within the same bound; the oracle runs in fp64 on the fp16 inputs."""
    case = prefill_case(lengths, seed=31, num_slots=6, Hk=2, Hv=4, g_scale=g_scale, dtype=torch.float16)
    o, st, o_ref, st_ref = _run(case, dev)
    assert o.dtype == torch.float16
    _check(case, o, st, o_ref, st_ref)


def test_prefill_fp16_matches_bf16_rounded_inputs(dev):
    """The same values through both kernels: bf16 inputs converted exactly to
    fp16 give the bf16 run's state to fp32 rounding and its output to bf16
    rounding."""
    case = prefill_case([130, 64], seed=32, num_slots=3, Hk=2, Hv=4)
    st_b, st_h = case.state.to(dev), case.state.to(dev)
    args = [t.to(dev) for t in (case.g, case.beta)]
    idx, cu = case.idx.to(dev), case.cu.to(dev)
    o_b = chunk_gated_delta_rule(case.q.to(dev), case.k.to(dev), case.v.to(dev), *args, st_b, idx, cu)
    o_h = chunk_gated_delta_rule(case.q.to(dev).half(), case.k.to(dev).half(), case.v.to(dev).half(), *args, st_h, idx, cu)
    torch.cuda.synchronize()
    assert o_h.dtype == torch.float16
    torch.testing.assert_close(o_h.float().cpu(), o_b.float().cpu(), rtol=1e-2, atol=1e-3)
    torch.testing.assert_close(st_h.cpu(), st_b.cpu(), rtol=1e-5, atol=1e-6)


def _stream_batch():
    """40 sequences of 0..150 tokens with a 0-, 1-, 64-, 65- and 300-token
    sequence and a padding slot among them (Hk 2 / Hv 4: 160 items)."""
    gen = torch.Generator().manual_seed(41)
    lengths = torch.randint(0, 151, (40,), generator=gen).tolist()
    lengths[3], lengths[5], lengths[9], lengths[10], lengths[11] = 0, 1, 64, 65, 300
    case = prefill_case(lengths, seed=42, num_slots=48, Hk=2, Hv=4)
    idx = case.idx.clone()
    idx[7] = -1
    return case, idx


@pytest.mark.parametrize("per_wg", [0, 1, 3, 64])
def test_prefill_item_stream(dev, per_wg):
    """The same batch with one item (sequence, v-head) per workgroup, longest
    first (0), and with runs of about 1, 3 and 64 items per workgroup (dealt
    by their token counts) walked as one chunk stream, whose producers stage
    the next item's first chunks while the state waves finish the current
    item."""
    case, idx = _stream_batch()
    print(f"prefill item stream: {per_wg} items per workgroup, {case.tokens} tokens", flush=True)
    o, st, o_ref, st_ref = _run(case, dev, idx=idx, items_per_wg=per_wg)
    _check(case, o, st, o_ref, st_ref, idx=idx)


def test_prefill_many_short_sequences_auto_stream(dev):
    """600 sequences of 1..128 tokens (2,400 items, under two chunks each on
    average): the launcher picks the chunk-stream schedule by itself."""
    gen = torch.Generator().manual_seed(43)
    lengths = torch.randint(1, 129, (600,), generator=gen).tolist()
    case = prefill_case(lengths, seed=44, num_slots=640, Hk=2, Hv=4)
    print(f"prefill many short sequences: {case.tokens} tokens", flush=True)
    o, st, o_ref, st_ref = _run(case, dev)
    _check(case, o, st, o_ref, st_ref)


def test_prefill_wait_give_up_poisons_the_stream(dev):
    """With several items per workgroup a wait that gives up poisons every
    item of the workgroup from that point: all rows NaN here (the limit is 0
    from the start), no state slot written."""
    case, idx = _stream_batch()
    o, st, _, _ = _run(case, dev, idx=idx, items_per_wg=8, spin_limit=0)
    pad = torch.zeros(case.tokens, dtype=torch.bool)
    pad[int(case.cu[7]):int(case.cu[8])] = True
    assert torch.isnan(o[~pad].float()).all()
    assert torch.count_nonzero(o[pad]) == 0
    assert torch.equal(st, case.state)


def test_prefill_wait_give_up_poisons_the_item(dev):
    """The kernel's waits between its wave roles are bounded; one that gives
    up must not pass as a plausible answer.  Forced from the host (spin limit
    0, so every wait gives up at once and every wave still runs to its end):
    every output row is NaN and no state slot is written.  With the default
    limit the same call is correct again."""
    case = prefill_case([200, 70], seed=25, num_slots=3, Hk=2, Hv=4)
    o, st, _, _ = _run(case, dev, spin_limit=0)
    assert torch.isnan(o.float()).all()
    assert torch.equal(st, case.state)
    o, st, o_ref, st_ref = _run(case, dev, spin_limit=-1)
    _check(case, o, st, o_ref, st_ref)


@pytest.mark.parametrize("lengths,g_scale", [([70, 5, 130, 1], 1.0), ([300, 1000], 0.02)])
def test_prefill_fp32_inputs(dev, lengths, g_scale):
    """fp32 q, k, v: q and k are rounded to fp16 (the MFMA operand type, the
    precision of the tf32 dots the reference's kernels run fp32 in) and v is
    carried as fp16 hi + lo through two launches.  Bars: the output against
    the oracle on the raw fp32 inputs within 1e-3 + 2e-3 |ref| (measured
    <= 0.07 of it); the state against the oracle fed the same fp16-rounded
    q and k within the usual 1e-3 |ref| + 1e-6 (measured <= 0.17 of it), and
    against the raw fp32 oracle within 1e-3 relative in norm (measured
    2.2e-4: the rounding of q and k).  A padding sequence and an untouched
    slot ride along."""
    N = len(lengths)
    case = prefill_case(lengths, seed=3, num_slots=N + 2, Hk=2, Hv=4, dtype=torch.float32, g_scale=g_scale)
    idx = case.idx.clone()
    idx[-1] = -1
    print(f"prefill fp32 inputs {lengths}", flush=True)
    o, st, o_raw, st_raw = _run(case, dev, idx=idx)
    assert o.dtype == torch.float32
    assert_out_close(o, o_raw, rtol=2e-3, atol=1e-3)
    s, e = int(case.cu[-2]), int(case.cu[-1])
    assert torch.count_nonzero(o[s:e]) == 0
    used = torch.tensor([int(i) for i in idx.tolist() if i >= 0], dtype=torch.long)
    st_r = case.state.clone()
    chunk_gated_delta_rule_ref(case.q.half().float(), case.k.half().float(), case.v, case.g, case.beta, st_r, idx,
                               case.cu)
    assert_state_close(st[used], st_r[used])
    rel = ((st[used].double() - st_raw[used]).norm() / st_raw[used].norm()).item()
    worst = ((st[used].double() - st_raw[used]).abs() / (1e-6 + 1e-3 * st_raw[used].abs())).max().item()
    print(f"prefill fp32 inputs {lengths}: state vs the raw fp32 oracle: relative norm {rel:.2e}, "
          f"worst element {worst:.2f} x the elementwise bar", flush=True)
    assert rel < 1e-3, rel
    untouched = torch.ones(N + 2, dtype=torch.bool)
    untouched[used] = False
    assert torch.equal(st[untouched], case.state[untouched])
