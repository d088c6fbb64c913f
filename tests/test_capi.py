"""CPU tests of the C ABI: the library loads, exports every declared symbol,
and rejects malformed calls before launching anything.

The validation calls use CPU tensors, so these tests are skipped where a GPU
is visible (a validation bug there would hand host pointers to a kernel);
the GPU tests cover the accepted paths.
"""
import os
import re

import pytest
import torch

from myvllm_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gdn_hip.h")

ERR = {"NULL": -1, "NDIM": -2, "SHAPE": -3, "DTYPE": -4, "STRIDE": -5, "HEADS": -6, "HEAD_DIM": -7, "CHUNK": -8,
       "ALIGN": -9, "CONV_WIDTH": -10, "RANGE": -11, "SCRATCH": -12, "ARG": -13}


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?(?:int64_t|int|char\s*\*|size_t|void)\s*\*?\s*(\w+)\s*\(", text, re.M)))


def test_header_declares_the_ffi_surface():
    assert declared_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.gdn_abi_version() == _lib.ABI_VERSION


def test_library_reads_no_environment():
    """Schedules and wait bounds are call arguments (gdn_chunk_prefill_ex),
    not environment variables: the built library imports no getenv, so a
    stray variable in a serving process cannot change a call."""
    import shutil
    import subprocess

    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm is not installed")
    undefined = subprocess.run([nm, "-D", "--undefined-only", _lib.LIB_PATH], check=True, capture_output=True,
                               text=True).stdout
    names = {line.split()[-1].split("@")[0] for line in undefined.splitlines() if line.strip()}
    assert "hipLaunchKernel" in names  # (the listing is the library's own imports)
    assert not names & {"getenv", "secure_getenv", "__secure_getenv"}, names


def test_header_error_codes_match():
    text = open(HEADER).read()
    for name, code in ERR.items():
        assert re.search(rf"#define GDN_ERR_{name} \({code}\)", text), name
    for code in list(ERR.values()) + [0]:
        assert _lib.strerror(code) != "unknown error code"
    assert _lib.strerror(-99) == "unknown error code"


cpu_only = pytest.mark.skipif(torch.cuda.is_available(), reason="validation tests hand CPU pointers to the C ABI")

D = _lib.describe


def _recurrent_args(B=2, Hk=2, Hv=4, K=128, V=128, slots=3, dtype=torch.bfloat16):
    return dict(
        q=torch.zeros(B, Hk, K, dtype=dtype), k=torch.zeros(B, Hk, K, dtype=dtype), v=torch.zeros(B, Hv, V, dtype=dtype),
        g=torch.zeros(B, Hv), beta=torch.zeros(B, Hv), state=torch.zeros(slots, Hv, K, V),
        idx=torch.zeros(B, dtype=torch.int32), out=torch.zeros(B, Hv, V, dtype=dtype),
    )


def _call_recurrent(a):
    lib = _lib.load()
    return lib.gdn_recurrent_step(D(a["q"]), D(a["k"]), D(a["v"]), D(a["g"]), D(a["beta"]), D(a["state"]),
                                  D(a["idx"]), D(a["out"]), 1.0, None)


def _call_prefill(a, cu, chunk=64):
    lib = _lib.load()
    return lib.gdn_chunk_prefill(D(a["q"]), D(a["k"]), D(a["v"]), D(a["g"]), D(a["beta"]), D(a["state"]),
                                 D(a["idx"]), D(cu), D(a["out"]), 1.0, chunk, None)


@cpu_only
@pytest.mark.parametrize(
    "mutate, code",
    [
        (lambda a: a.update(g=torch.zeros(2, 4, 1)), "NDIM"),
        (lambda a: a.update(v=torch.zeros(3, 4, 128, dtype=torch.bfloat16)), "SHAPE"),
        (lambda a: a.update(state=torch.zeros(3, 2, 128, 128)), "SHAPE"),
        (lambda a: a.update(idx=torch.zeros(3, dtype=torch.int32)), "SHAPE"),
        (lambda a: a.update(v=torch.zeros(2, 3, 128, dtype=torch.bfloat16), out=torch.zeros(2, 3, 128, dtype=torch.bfloat16),
                            g=torch.zeros(2, 3), beta=torch.zeros(2, 3), state=torch.zeros(3, 3, 128, 128)), "HEADS"),
        (lambda a: a.update(out=torch.zeros(2, 4, 128, dtype=torch.float32)), "DTYPE"),
        (lambda a: a.update(state=torch.zeros(3, 4, 128, 128, dtype=torch.bfloat16)), "DTYPE"),
        (lambda a: a.update(idx=torch.zeros(2, dtype=torch.float32)), "DTYPE"),
        (lambda a: a.update(q=torch.zeros(2, 2, 256, dtype=torch.bfloat16)[:, :, ::2]), "STRIDE"),
        (lambda a: a.update(state=torch.zeros(3, 4, 128, 256)[..., :128]), "STRIDE"),
        (lambda a: a.update(**_recurrent_args(K=100, V=96)), "HEAD_DIM"),
        (lambda a: a.update(**_recurrent_args(K=264, V=128)), "HEAD_DIM"),
        (lambda a: a.update(**_recurrent_args(K=128, V=260)), "HEAD_DIM"),
    ],
)
def test_recurrent_step_validation(mutate, code):
    a = _recurrent_args()
    mutate(a)
    assert _call_recurrent(a) == ERR[code]


@cpu_only
def test_recurrent_step_null_descriptor():
    a = _recurrent_args()
    lib = _lib.load()
    rc = lib.gdn_recurrent_step(None, D(a["k"]), D(a["v"]), D(a["g"]), D(a["beta"]), D(a["state"]), D(a["idx"]),
                                D(a["out"]), 1.0, None)
    assert rc == ERR["NULL"]


@cpu_only
def test_prefill_validation():
    a = _recurrent_args(B=10)
    a["idx"] = torch.zeros(2, dtype=torch.int32)
    cu = torch.tensor([0, 4, 10], dtype=torch.int32)
    assert _call_prefill(a, cu, chunk=32) == ERR["CHUNK"]
    assert _call_prefill(a, torch.tensor([0, 10], dtype=torch.int32)) == ERR["SHAPE"]  # idx has 2 entries
    b = _recurrent_args(B=10, dtype=torch.float32)
    b["idx"] = torch.zeros(2, dtype=torch.int32)
    assert _call_prefill(b, cu) == ERR["DTYPE"]  # prefill takes bf16 or fp16 q/k/v only
    for K, V in ((100, 64), (136, 128), (128, 4), (0, 64)):  # head dims: multiples of 8 in 8..128
        c = _recurrent_args(B=10, K=K, V=V)
        c["idx"] = torch.zeros(2, dtype=torch.int32)
        assert _call_prefill(c, cu) == ERR["HEAD_DIM"], (K, V)
    d = _recurrent_args(B=10)
    d["idx"] = torch.zeros(2, dtype=torch.int32)
    d["g"] = torch.zeros(10, 4, dtype=torch.bfloat16)
    assert _call_prefill(d, cu) == ERR["DTYPE"]


def _call_prefill_ex(a, cu, flags=0, per_wg=-1, spin=-1):
    lib = _lib.load()
    return lib.gdn_chunk_prefill_ex(D(a["q"]), D(a["k"]), D(a["v"]), D(a["g"]), D(a["beta"]), D(a["state"]),
                                    D(a["idx"]), D(cu), D(a["out"]), 1.0, 64, flags, per_wg, spin, None)


@cpu_only
def test_prefill_ex_validation():
    """gdn_chunk_prefill_ex: unknown flags and out-of-range options are
    GDN_ERR_ARG; an fp32 out only for fp16 q/k/v, and ACCUM_OUT only with it;
    everything else is checked as for gdn_chunk_prefill."""
    a = _recurrent_args(B=10)
    a["idx"] = torch.zeros(2, dtype=torch.int32)
    cu = torch.tensor([0, 4, 10], dtype=torch.int32)
    assert _call_prefill_ex(a, cu, flags=8) == ERR["ARG"]
    assert _call_prefill_ex(a, cu, per_wg=65) == ERR["ARG"]
    assert _call_prefill_ex(a, cu, per_wg=-2) == ERR["ARG"]
    assert _call_prefill_ex(a, cu, spin=-2) == ERR["ARG"]
    assert _call_prefill_ex(a, cu, spin=(1 << 22) + 1) == ERR["ARG"]
    assert _call_prefill_ex(a, cu, flags=_lib.PREFILL_ACCUM_OUT) == ERR["DTYPE"]  # bf16 out
    a["out"] = torch.zeros(10, 4, 128, dtype=torch.float32)
    assert _call_prefill_ex(a, cu) == ERR["DTYPE"]  # fp32 out needs fp16 inputs
    b = _recurrent_args(B=10, dtype=torch.float16)
    b["idx"] = torch.zeros(2, dtype=torch.int32)
    b["out"] = torch.zeros(10, 4, 100, dtype=torch.float32)
    assert _call_prefill_ex(b, cu) == ERR["SHAPE"]
    e = _recurrent_args(B=10)
    e["idx"] = torch.zeros(2, dtype=torch.int32)
    e["v"] = torch.zeros(10, 4, 130, dtype=torch.bfloat16)[:, :, 1:129]  # 2-byte offset: misaligned
    assert _call_prefill(e, cu) == ERR["ALIGN"]


def _conv_args(T=6, D_=64, W=4, slots=3, N=2):
    return dict(x=torch.zeros(T, D_, dtype=torch.bfloat16), w=torch.zeros(D_, W, dtype=torch.bfloat16),
                st=torch.zeros(slots, W - 1, D_), idx=torch.zeros(N, dtype=torch.int32),
                cu=torch.tensor([0, 2, T], dtype=torch.int32), out=torch.zeros(T, D_, dtype=torch.bfloat16))


def _call_conv(a):
    return _lib.load().causal_conv1d_varlen(D(a["x"]), D(a["w"]), D(a["st"]), D(a["idx"]), D(a["cu"]), D(a["out"]),
                                            None)


@cpu_only
@pytest.mark.parametrize(
    "mutate, code",
    [
        (lambda a: a.update(w=torch.zeros(64, 7, dtype=torch.bfloat16), st=torch.zeros(3, 6, 64)), "CONV_WIDTH"),
        (lambda a: a.update(w=torch.zeros(64, 1, dtype=torch.bfloat16), st=torch.zeros(3, 0, 64)), "CONV_WIDTH"),
        (lambda a: a.update(st=torch.zeros(3, 2, 64)), "SHAPE"),
        (lambda a: a.update(x=torch.zeros(6, 60, dtype=torch.bfloat16), w=torch.zeros(60, 4, dtype=torch.bfloat16),
                            st=torch.zeros(3, 3, 60), out=torch.zeros(6, 60, dtype=torch.bfloat16)), "SHAPE"),
        (lambda a: a.update(out=torch.zeros(6, 64)), "DTYPE"),
        (lambda a: a.update(w=torch.zeros(64, 4, dtype=torch.float16)), "DTYPE"),
        (lambda a: a.update(cu=torch.zeros(3, dtype=torch.float32)), "DTYPE"),
        (lambda a: a.update(x=torch.zeros(64, 6, dtype=torch.bfloat16).t()), "STRIDE"),
        (lambda a: a.update(x=torch.zeros(6, 72, dtype=torch.bfloat16)[:, 4:68]), "ALIGN"),
    ],
)
def test_conv_validation(mutate, code):
    a = _conv_args()
    mutate(a)
    assert _call_conv(a) == ERR[code]


@cpu_only
def test_conv_step_validation():
    lib = _lib.load()
    x = torch.zeros(3, 64, dtype=torch.bfloat16)
    rc = lib.causal_conv1d_step(D(x), D(torch.zeros(64, 4, dtype=torch.bfloat16)), D(torch.zeros(4, 3, 64)),
                                D(torch.zeros(2, dtype=torch.int32)), D(torch.zeros(3, 64, dtype=torch.bfloat16)), None)
    assert rc == ERR["SHAPE"]  # 3 tokens, 2 slot indices


def _fused_args(B=2, Hk=2, Hv=4, K=128, V=128, slots=3, dtype=torch.bfloat16):
    Dc = 2 * Hk * K + Hv * V
    return dict(
        x=torch.zeros(B, Dc, dtype=dtype), w=torch.zeros(Dc, 4, dtype=dtype), cs=torch.zeros(slots, 3, Dc),
        cidx=torch.zeros(B, dtype=torch.int32), a=torch.zeros(B, Hv, dtype=dtype), b=torch.zeros(B, Hv, dtype=dtype),
        A_log=torch.zeros(Hv), dt_bias=torch.zeros(Hv), state=torch.zeros(slots, Hv, K, V),
        idx=torch.zeros(B, dtype=torch.int32), out=torch.zeros(B, Hv, V, dtype=dtype), Hk=Hk,
    )


def _call_fused(a):
    lib = _lib.load()
    return lib.gdn_decode_step_fused(D(a["x"]), D(a["w"]), D(a["cs"]), D(a["cidx"]), D(a["a"]), D(a["b"]),
                                     D(a["A_log"]), D(a["dt_bias"]), D(a["state"]), D(a["idx"]), D(a["out"]),
                                     a["Hk"], 0.1, None)


@cpu_only
@pytest.mark.parametrize(
    "mutate,code",
    [
        (lambda a: a.update(w=torch.zeros(1024, 3, dtype=torch.bfloat16)), "CONV_WIDTH"),
        (lambda a: a.update(Hk=3), "HEADS"),
        (lambda a: a.update(Hk=0), "HEADS"),
        (lambda a: a.update(x=torch.zeros(2, 1000, dtype=torch.bfloat16)), "SHAPE"),
        (lambda a: a.update(cs=torch.zeros(3, 2, 1024)), "SHAPE"),
        (lambda a: a.update(cs=torch.zeros(0, 3, 1024)), "SHAPE"),
        (lambda a: a.update(state=torch.zeros(0, 4, 128, 128)), "SHAPE"),
        (lambda a: a.update(cidx=torch.zeros(3, dtype=torch.int32)), "SHAPE"),
        (lambda a: a.update(a=torch.zeros(2, 3, dtype=torch.bfloat16)), "SHAPE"),
        (lambda a: a.update(A_log=torch.zeros(5)), "SHAPE"),
        (lambda a: a.update(out=torch.zeros(2, 4, 128)), "DTYPE"),
        (lambda a: a.update(state=torch.zeros(3, 4, 128, 128, dtype=torch.float16)), "DTYPE"),
        (lambda a: a.update(idx=torch.zeros(2, dtype=torch.float32)), "DTYPE"),
        (lambda a: a.update(state=torch.zeros(3, 4, 64, 64), x=torch.zeros(2, 512, dtype=torch.bfloat16),
                            w=torch.zeros(512, 4, dtype=torch.bfloat16), cs=torch.zeros(3, 3, 512),
                            out=torch.zeros(2, 4, 64, dtype=torch.bfloat16)), "HEAD_DIM"),
        (lambda a: a.update(x=torch.zeros(1024, 2, dtype=torch.bfloat16).t()), "STRIDE"),
        (lambda a: a.update(cidx=torch.zeros(4, dtype=torch.int32)[::2]), "STRIDE"),
        (lambda a: a.update(state=torch.zeros(3 * 4 * 128 * 128 + 1)[1:].view(3, 4, 128, 128)), "ALIGN"),
    ],
)
def test_fused_decode_validation(mutate, code):
    a = _fused_args()
    mutate(a)
    assert _call_fused(a) == ERR[code]


@cpu_only
def test_fused_decode_heads_ratio_eight_rejected():
    a = _fused_args(Hk=1, Hv=8)
    assert _call_fused(a) == ERR["HEADS"]


def test_ops_reject_cpu_tensors():
    from myvllm_amd import causal_conv1d_update, recurrent_gated_delta_rule

    a = _recurrent_args()
    with pytest.raises(ValueError):
        recurrent_gated_delta_rule(a["q"], a["k"], a["v"], a["g"], a["beta"], a["state"], a["idx"])
    c = _conv_args()
    with pytest.raises(ValueError):
        causal_conv1d_update(c["x"][:2], c["w"], c["st"], c["idx"])


# ---- full attention ------------------------------------------------------------------

def _varlen_attn_args(T=8, Hq=4, Hkv=2, Dh=128, dtype=torch.bfloat16):
    return dict(q=torch.zeros(T, Hq, Dh, dtype=dtype), k=torch.zeros(T, Hkv, Dh, dtype=dtype),
                v=torch.zeros(T, Hkv, Dh, dtype=dtype), cu=torch.tensor([0, 3, T], dtype=torch.int32),
                out=torch.zeros(T, Hq, Dh, dtype=dtype), max_len=5)


def _call_varlen_attn(a):
    return _lib.load().flash_attention_varlen(D(a["q"]), D(a["k"]), D(a["v"]), D(a["cu"]), D(a["out"]),
                                              a["max_len"], 1.0, 1, None)


@cpu_only
@pytest.mark.parametrize(
    "mutate, code",
    [
        (lambda a: a.update(q=torch.zeros(8, 4, 128, 1, dtype=torch.bfloat16)), "NDIM"),
        (lambda a: a.update(k=torch.zeros(7, 2, 128, dtype=torch.bfloat16)), "SHAPE"),
        (lambda a: a.update(v=torch.zeros(8, 1, 128, dtype=torch.bfloat16)), "SHAPE"),
        (lambda a: a.update(out=torch.zeros(8, 4, 64, dtype=torch.bfloat16)), "SHAPE"),
        (lambda a: a.update(max_len=-1), "SHAPE"),
        (lambda a: a.update(q=torch.zeros(8, 3, 128, dtype=torch.bfloat16), out=torch.zeros(8, 3, 128, dtype=torch.bfloat16)), "HEADS"),
        (lambda a: a.update(q=torch.zeros(8, 4, 128), out=torch.zeros(8, 4, 128)), "DTYPE"),
        (lambda a: a.update(v=torch.zeros(8, 2, 128, dtype=torch.float16)), "DTYPE"),
        (lambda a: a.update(cu=torch.tensor([0.0, 8.0])), "DTYPE"),
        (lambda a: a.update(q=torch.zeros(8, 4, 96, dtype=torch.bfloat16), k=torch.zeros(8, 2, 96, dtype=torch.bfloat16),
                            v=torch.zeros(8, 2, 96, dtype=torch.bfloat16), out=torch.zeros(8, 4, 96, dtype=torch.bfloat16)), "HEAD_DIM"),
        (lambda a: a.update(k=torch.zeros(8, 128, 2, dtype=torch.bfloat16).transpose(1, 2)), "STRIDE"),
        (lambda a: a.update(q=torch.zeros(8 * 4 * 128 + 1, dtype=torch.bfloat16)[1:].view(8, 4, 128)), "ALIGN"),
    ],
)
def test_varlen_attention_validation(mutate, code):
    a = _varlen_attn_args()
    mutate(a)
    assert _call_varlen_attn(a) == ERR[code]


@cpu_only
@pytest.mark.parametrize("max_len, code", [(5, "RANGE"), (2**20, "RANGE")])
def test_varlen_attention_key_tile_range(max_len, code):
    """A 64-row key tile of k or v must span less than 2^31 bytes whatever
    max_seqlen says (2^24-element rows: 5 rows fit, 64 do not)."""
    a = _varlen_attn_args()
    k = D(a["k"])
    k.stride[0] = 2**24
    rc = _lib.load().flash_attention_varlen(D(a["q"]), k, D(a["v"]), D(a["cu"]), D(a["out"]), max_len, 1.0, 1, None)
    assert rc == ERR[code]


def _paged_attn_args(B=2, Hq=4, Hkv=2, Dh=128, blocks=5, page=16, cols=3, dtype=torch.bfloat16):
    return dict(q=torch.zeros(B, Hq, Dh, dtype=dtype), kc=torch.zeros(blocks, page, Hkv, Dh, dtype=dtype),
                vc=torch.zeros(blocks, page, Hkv, Dh, dtype=dtype), tab=torch.zeros(B, cols, dtype=torch.int32),
                ctx=torch.ones(B, dtype=torch.int32), out=torch.zeros(B, Hq, Dh, dtype=dtype),
                ws=torch.zeros(_lib.load().paged_attention_decode_workspace_size(B, Hq, Dh, 4)), splits=4)


def _call_paged_decode(a):
    return _lib.load().paged_attention_decode(D(a["q"]), D(a["kc"]), D(a["vc"]), D(a["tab"]), D(a["ctx"]),
                                              D(a["out"]), D(a["ws"]) if a["ws"] is not None else None,
                                              a["splits"], 1.0, None)


@cpu_only
@pytest.mark.parametrize(
    "mutate, code",
    [
        (lambda a: a.update(kc=torch.zeros(5, 16, 256, dtype=torch.bfloat16)), "NDIM"),
        (lambda a: a.update(vc=torch.zeros(4, 16, 2, 128, dtype=torch.bfloat16)), "SHAPE"),
        (lambda a: a.update(tab=torch.zeros(3, 3, dtype=torch.int32)), "SHAPE"),
        (lambda a: a.update(ctx=torch.zeros(3, dtype=torch.int32)), "SHAPE"),
        (lambda a: a.update(ws=torch.zeros(10)), "SHAPE"),
        (lambda a: a.update(ws=None), "NULL"),
        (lambda a: a.update(ws=torch.zeros(a["ws"].numel(), dtype=torch.float16)), "DTYPE"),
        (lambda a: a.update(tab=torch.zeros(2, 3)), "DTYPE"),
        (lambda a: a.update(tab=torch.zeros(3, 2, dtype=torch.int32).t()), "STRIDE"),
        (lambda a: a.update(splits=0), "RANGE"),
        (lambda a: a.update(splits=257), "RANGE"),
        (lambda a: a.update(ws=torch.zeros(a["ws"].numel() + 1)[1:]), "ALIGN"),
    ],
)
def test_paged_decode_validation(mutate, code):
    a = _paged_attn_args()
    mutate(a)
    assert _call_paged_decode(a) == ERR[code]


@cpu_only
def test_paged_prefill_validation():
    a = _paged_attn_args()
    q = torch.zeros(5, 4, 128, dtype=torch.bfloat16)
    cu = torch.tensor([0, 2, 5], dtype=torch.int32)

    def call(q=q, cu=cu, out=None, tab=a["tab"], ctx=a["ctx"], max_len=3):
        out = torch.zeros_like(q) if out is None else out
        return _lib.load().paged_attention_prefill(D(q), D(a["kc"]), D(a["vc"]), D(tab), D(ctx), D(cu), D(out),
                                                   max_len, 1.0, None)

    assert call(cu=torch.tensor([0, 5], dtype=torch.int32)) == ERR["SHAPE"]  # one sequence, two table rows
    assert call(out=torch.zeros(5, 4, 256, dtype=torch.bfloat16)) == ERR["SHAPE"]
    assert call(max_len=-1) == ERR["SHAPE"]
    assert call(ctx=torch.ones(2)) == ERR["DTYPE"]
    assert call(cu=torch.tensor([0.0, 2.0, 5.0])) == ERR["DTYPE"]


@cpu_only
@pytest.mark.parametrize("cols, splits, refused", [(2**30, 4, True), (2**30, 1, False), (2**29 - 4, 4, False)])
def test_paged_decode_price_range(cols, splits, refused):
    """The split decode prices the batch (16-key tiles of the table's capacity
    plus a start price of 2 per sequence) in 32 bits: 2 sequences x 2^30
    columns of 16 keys exceed 2^31 and are refused (RANGE) before any HIP
    call; 2^29 - 4 columns fit, and one split prices nothing (on a machine
    without a GPU those calls get as far as the launch, which fails).  Only
    the descriptor's column count is large: no kernel runs."""
    a = _paged_attn_args()
    a["splits"] = splits
    tab = D(a["tab"])
    tab.shape[1] = cols
    rc = _lib.load().paged_attention_decode(D(a["q"]), D(a["kc"]), D(a["vc"]), tab, D(a["ctx"]), D(a["out"]),
                                            D(a["ws"]), splits, 1.0, None)
    assert (rc == ERR["RANGE"]) == refused
    if not refused:
        assert rc > 0  # a hipError_t from the launch


@pytest.mark.parametrize(
    "B, Hq, Hkv, capacity, splits",
    [
        (256, 16, 2, 4096, 2),     # 512 (sequence, kv head) rows: one unit per sequence
        (128, 16, 2, 4096, 3),     # 256 rows: two units per sequence
        (64, 16, 2, 32768, 5),     # 128 rows: four
        (16, 16, 2, 32768, 17),    # 32 rows: sixteen
        (512, 16, 2, 2048, 2),     # 1,024 rows: still at least one unit per sequence
        (1024, 16, 2, 1024, 1),    # 2,048 rows: one split
        (1, 64, 2, 100000, 129),   # 32 query heads per kv head: two head groups, 4 rows, 128 units
        (3, 16, 2, 300, 3),        # capacity 300: at most ceil(300 / 256) = 2 units per sequence
        (1, 16, 1, 10**6, 256),    # the cap
    ],
)
def test_decode_num_splits(B, Hq, Hkv, capacity, splits):
    """The decode's default split count: about 512 unit x kv head x head
    group waves, at least one unit per sequence below 2,048 rows, one split
    from there, at most ceil(capacity / 256) units per sequence and 256
    splits."""
    from myvllm_amd.full_attention import decode_num_splits
    assert decode_num_splits(B, Hq, Hkv, capacity) == splits


def test_decode_workspace_size():
    lib = _lib.load()
    assert lib.paged_attention_decode_workspace_size(3, 16, 256, 1) == 0
    assert lib.paged_attention_decode_workspace_size(3, 16, 256, 4) == 3 * 4 * 16 * 260 + 4


def _call_paged_decode_noalloc(a):
    return _lib.load().paged_attention_decode_noalloc(D(a["q"]), D(a["kc"]), D(a["vc"]), D(a["tab"]), D(a["ctx"]),
                                                      D(a["out"]), a["splits"], 1.0, None)


@cpu_only
def test_paged_decode_noalloc_validation():
    a = _paged_attn_args()
    a.update(kc=torch.zeros(5, 16, 256, dtype=torch.bfloat16))
    assert _call_paged_decode_noalloc(a) == ERR["NDIM"]
    a = _paged_attn_args()
    a.update(splits=257)
    assert _call_paged_decode_noalloc(a) == ERR["RANGE"]
    a = _paged_attn_args()
    a.update(tab=torch.zeros(3, 2, dtype=torch.int32).t())
    assert _call_paged_decode_noalloc(a) == ERR["STRIDE"]


@cpu_only
def test_paged_decode_noalloc_rejects_more_than_the_static_scratch():
    # 64 sequences x 64 query heads x 256 splits x (256 + 4) fp32 partials > GDN_DECODE_SCRATCH_FLOATS
    B, Hq, Hkv, Dh = 64, 64, 8, 256
    a = dict(q=torch.zeros(B, Hq, Dh, dtype=torch.bfloat16), kc=torch.zeros(4, 16, Hkv, Dh, dtype=torch.bfloat16),
             vc=torch.zeros(4, 16, Hkv, Dh, dtype=torch.bfloat16), tab=torch.zeros(B, 4, dtype=torch.int32),
             ctx=torch.ones(B, dtype=torch.int32), out=torch.zeros(B, Hq, Dh, dtype=torch.bfloat16), splits=256)
    text = open(HEADER).read()
    cap = eval(re.search(r"#define GDN_DECODE_SCRATCH_FLOATS \(([^)]*)\)", text).group(1))
    assert _lib.load().paged_attention_decode_workspace_size(B, Hq, Dh, 256) > cap
    assert _call_paged_decode_noalloc(a) == ERR["SCRATCH"]
    a["splits"] = 1  # no partials: nothing needs the scratch
    assert _lib.load().paged_attention_decode_workspace_size(B, Hq, Dh, 1) == 0



@cpu_only
def test_rms_norm_gated_validation():
    """Any row length N; weight (N,) or (H, N); shapes must agree."""
    lib = _lib.load()
    x = torch.zeros(3, 2, 72, dtype=torch.bfloat16)

    def call(x, g, w, o):
        return lib.gdn_rms_norm_gated(D(x), D(g), D(w), D(o), 1e-6, None)

    assert call(x, x, torch.ones(71), x) == ERR["SHAPE"]
    assert call(x, x, torch.ones(3, 72), x) == ERR["SHAPE"]  # per-head weight with 3 rows for 2 heads
    assert call(x, torch.zeros(3, 2, 72), torch.ones(72), x) == ERR["DTYPE"]
    assert call(x, x, torch.ones(72, 2)[:, 0], x) == ERR["STRIDE"]
    assert call(x, x, torch.ones(1, 2, 72), x) == ERR["NDIM"]
