"""bench.py's command line on the CPU: it measures one GPU only and refuses
more, and it rejects unknown workloads and invalid step counts, before
touching a device."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120)


def test_more_than_one_gpu_exits_with_a_message():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_world_size_above_one_exits_too():
    env = dict(os.environ, WORLD_SIZE="2")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")], capture_output=True, text=True, timeout=120,
                       env=env)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_invalid_step_counts_are_refused():
    for args in (("--steps", "0"), ("--warmup", "-1"), ("--settle-ms", "-5")):
        r = _run(*args)
        assert r.returncode == 2 and "--steps must be at least 1" in r.stderr, args


def test_traffic_table_matches_the_committed_profiles():
    """bench.py reports roofline.traffic from its HBM_TRAFFIC_PER_LAUNCH table
    (the GPU box has no profiles/ directory to read it from); every entry
    must equal the "traffic per launch" line of the profile summary it was
    taken from, so a re-profiled kernel cannot leave a stale figure behind."""
    import re

    sys.path.insert(0, ROOT)
    import bench

    sources = {
        "gdn_chunk_prefill_kernel": "gdn_chunk_prefill_kernel__prefill_32k_varlen.md",
        "gdn_chunk_prefill_kernel/short": "gdn_chunk_prefill_kernel__prefill_short_512x64.md",
        "gdn_recurrent_step_kernel": "gdn_recurrent_step_kernel__decode_b256.md",
        "causal_conv1d_varlen_kernel": "causal_conv1d_varlen_kernel__conv_8seq_19762tok.md",
        "causal_conv1d_step_kernel": "causal_conv1d_step_kernel__conv_update_b256.md",
        "gdn_decode_fused_kernel": "gdn_decode_fused_kernel__decode_fused_b256.md",
        "attn_prefill_kernel": "attn_prefill_kernel__attn_prefill_16seq_35846tok_d256.md",
        "attn_decode_kernel": "attn_decode_kernel__attn_decode_b256_d256.md",
        "attn_paged_prefill_kernel": "attn_prefill_kernel__attn_paged_prefill_16seq_19041tok_d256.md",
    }
    assert set(sources) == set(bench.HBM_TRAFFIC_PER_LAUNCH)
    for key, fname in sources.items():
        text = open(os.path.join(ROOT, "profiles", fname)).read()
        m = re.search(r"traffic per launch: ([\d,]+) B", text)
        assert m, fname
        assert bench.HBM_TRAFFIC_PER_LAUNCH[key] == int(m.group(1).replace(",", "")), (key, fname)
