"""The decode launch's own merge of split rows against the merge launch.

For decode launches whose split rows have at most eight splits and whose KV
heads number a multiple of 8, the planner (capi.cpp: decode_merge_fusable,
choose_decode_rounds, decode_launch_us) lets the last split of each (row, kv
head) fold the records inside the decode launch, on the XCD where all of that
group's splits ran (decode.hip: merge_in_launch), instead of a merge launch.
The fold reproduces merge.hip's one-thread-per-(vector, 4 features) layout and
arithmetic, so the outputs must not depend on the path.

Each case runs in two fresh processes, one of them with
XINFER_DECODE_MERGE_LAUNCH=1 (every split row through the merge launch).  The
outputs must be equal bit for bit, the kernels each process launched
(torch.profiler) must show the path the case expects, and the outputs must
pass the float64 oracle's gates; keys past each row's length and queries past
its count are NaN, so a read outside them poisons the output.  The default
process also replays a captured graph of one case three times, with eager
work in between (the arrival counters must be back at zero after every
launch, since a replay reuses its launch's tag), and runs a case on a second
stream.
"""

import json
import os
from pathlib import Path
import subprocess
import sys
import textwrap

import numpy as np
import pytest
import torch

from attn_helpers import MAX_ABS, MEAN_ABS, log, row_errors
from oracle import attention as oracle

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]

# (name, Hq, Hkv, D, counts, lengths, capacity, path the planner takes).
# Keys per one-round item: 128 for head dim 128 with 1-4 query vectors per KV
# head, 256 for head dim 64, 64 for head dim 256 and for 8 query vectors.
CASES = [
    ("cfg1_shape", 16, 8, 128, [1], [1024], 4096, "in_launch"),          # 8 splits per kv head
    ("dim64_row", 16, 8, 64, [1], [1000], 2048, "in_launch"),           # 4 splits
    ("dim256_row", 16, 8, 256, [1], [512], 1024, "in_launch"),          # 8 splits
    ("dim72_padded", 16, 8, 72, [1, 1], [700, 33], 1024, "in_launch"),  # 6 and 1 splits
    ("rows_g1_empty", 8, 8, 128, [1, 1, 0, 1], [1024, 5, 3, 300], 2048, "in_launch"),
    ("group4_two_queries", 32, 8, 128, [2, 1, 2], [500, 512, 130], 1024, "in_launch"),  # 8 query vectors
    ("eight_short_rows", 16, 8, 128, [1] * 8, [1024, 1000, 900, 800, 700, 129, 64, 1], 2048, "in_launch"),
    # cfg3 seed 3's lengths: four-round items (512 keys) bring the longest
    # row to 7 splits, and the cost model takes them with the in-launch merge.
    ("cfg3_seed3_lengths", 16, 8, 128, [1] * 8, [20, 116, 3394, 53, 3006, 1084, 63, 322], 4096, "in_launch"),
    # Past eight splits, and KV heads not a multiple of 8: the merge launch.
    ("nine_splits", 16, 8, 128, [1], [1100], 2048, "merge"),
    ("four_kv_heads", 16, 4, 128, [1], [1024], 2048, "merge"),
]

CHILD = textwrap.dedent(
    """
    import json, sys
    import torch
    sys.path.insert(0, sys.argv[1])
    sys.path.insert(0, sys.argv[1] + '/tests')
    from test_decode_merge_gpu import CASES, make_case
    from xinfer_amd.attention import load_attention_ops, batched_attention_metadata
    load_attention_ops(model='qwen3')
    ops = torch.ops.xinfer
    outputs, report = {}, {}
    with torch.inference_mode():
        for name, heads, kv_heads, dim, counts, lengths, capacity, _ in CASES:
            print(name, file=sys.stderr, flush=True)
            q, k, v = (t.cuda() for t in make_case(name, heads, kv_heads, dim, counts, lengths, capacity))
            host, cu, blocks = batched_attention_metadata(torch.tensor(lengths, dtype=torch.int32),
                                                          torch.tensor(counts, dtype=torch.int32), 'cuda')
            scale = dim ** -0.5
            ops.batched_flash_attention(q, k, v, host, cu, blocks, scale)  # first call (runs the XCD probe)
            torch.cuda.synchronize()
            with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
                out = ops.batched_flash_attention(q, k, v, host, cu, blocks, scale)
                torch.cuda.synchronize()
            kernels = sorted({e.name.split('(')[0].split('<')[0] for e in prof.events() if 'xattn::' in e.name})
            outputs[name] = out.cpu()
            report[name] = dict(kernels=kernels)
            if name == 'cfg1_shape' and sys.argv[3] == 'default':
                graph = torch.cuda.CUDAGraph()
                captured = torch.empty_like(out)
                side = torch.cuda.Stream()
                side.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(side):
                    ops.batched_flash_attention(q, k, v, host, cu, blocks, scale)
                torch.cuda.current_stream().wait_stream(side)
                with torch.cuda.graph(graph):
                    captured.copy_(ops.batched_flash_attention(q, k, v, host, cu, blocks, scale))
                for replay in range(3):
                    captured.fill_(float('nan'))
                    graph.replay()
                    _ = ops.batched_flash_attention(q, k, v, host, cu, blocks, scale)  # eager call between replays
                    torch.cuda.synchronize()
                    if not torch.equal(captured.view(torch.int16), out.view(torch.int16)):
                        raise AssertionError(f'graph replay {replay} differs')
                other = torch.cuda.Stream()
                with torch.cuda.stream(other):
                    again = ops.batched_flash_attention(q, k, v, host, cu, blocks, scale)
                torch.cuda.synchronize()
                if not torch.equal(again.view(torch.int16), out.view(torch.int16)):
                    raise AssertionError('second stream differs')
                report[name]['graph_replays'] = 3
    torch.save(outputs, sys.argv[2])
    print(json.dumps(report), flush=True)
    """
)


def make_case(name, heads, kv_heads, dim, counts, lengths, capacity):
    """Seeded CPU bf16 inputs; NaN past each row's length (K, V) and count (Q)."""
    generator = torch.Generator().manual_seed(sum(map(ord, name)))
    batch, tokens = len(counts), max(counts)
    q = torch.randn(batch, heads, tokens, dim, generator=generator).to(torch.bfloat16)
    k = torch.randn(batch, kv_heads, capacity, dim, generator=generator).to(torch.bfloat16)
    v = torch.randn(batch, kv_heads, capacity, dim, generator=generator).to(torch.bfloat16)
    for r, (count, length) in enumerate(zip(counts, lengths)):
        k[r, :, length:] = float("nan")
        v[r, :, length:] = float("nan")
        q[r, :, count:] = float("nan")
    return q, k, v


def run_child(tmp_path, mode):
    target = tmp_path / f"{mode}.pt"
    env = dict(os.environ)
    env.pop("XINFER_DECODE_MERGE_LAUNCH", None)
    if mode == "merge_launch":
        env["XINFER_DECODE_MERGE_LAUNCH"] = "1"
    log(f"decode merge paths: {mode} process")
    result = subprocess.run([sys.executable, "-c", CHILD, str(ROOT), str(target), mode], env=env,
                            capture_output=True, text=True, timeout=600)
    assert result.returncode == 0, result.stdout[-3000:] + result.stderr[-3000:]
    return torch.load(target, weights_only=True), json.loads(result.stdout.splitlines()[-1])


def f64(tensor):
    return tensor.float().numpy().astype(np.float64)


def test_in_launch_merge_equals_the_merge_launch(gpu_ops, tmp_path):
    default, default_report = run_child(tmp_path, "default")
    forced, forced_report = run_child(tmp_path, "merge_launch")
    assert default_report["cfg1_shape"].get("graph_replays") == 3
    for name, heads, kv_heads, dim, counts, lengths, capacity, path in CASES:
        log(f"decode merge paths: {name} ({path})")
        kernels = default_report[name]["kernels"]
        assert any("decode_kernel" in kernel for kernel in kernels), kernels
        assert ("merge_kernel" in " ".join(kernels)) == (path == "merge"), (name, kernels)
        assert "merge_kernel" in " ".join(forced_report[name]["kernels"]), name
        out = default[name]
        assert torch.equal(out.view(torch.int16), forced[name].view(torch.int16)), name
        q, k, v = make_case(name, heads, kv_heads, dim, counts, lengths, capacity)
        expected = oracle.attention(*(f64(torch.nan_to_num(x, nan=0.0)) for x in (q, k, v)), counts, lengths,
                                    dim ** -0.5)
        for r, count in enumerate(counts):
            assert torch.count_nonzero(out[r, :, count:]).item() == 0
            if not count:
                continue
            errors = row_errors(out[r : r + 1, :, :count].float().flatten(1),
                                torch.from_numpy(expected[r : r + 1, :, :count]).float().flatten(1))
            assert errors["max_abs"] <= MAX_ABS and errors["mean_abs"] <= MEAN_ABS, (name, r, errors)
            assert errors["relative_l2"] < 0.01 and errors["peak_relative"] <= 0.05, (name, r, errors)
