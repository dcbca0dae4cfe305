"""bench.py's contract on the CPU: one GPU only (any other --gpus exits with a message before touching a device),
one workload per configuration, and the algorithmic bytes per parameter of the two kinds of step (norm 4 + Adam 30
with fp32 gradients; owner sum 18 + Adam 28 with bf16 ones)."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, 'bench.py'), '--gpus', '2'], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert 'one GPU only' in r.stderr and r.stdout == ''


def test_workloads_cover_every_config(pkg):
    from faster_yoco_amd import configs
    assert set(bench.WORKLOADS) == set(configs.CONFIGS)


def test_algorithmic_bytes():
    n = 430_662_912
    assert bench.algorithmic_bytes('c2', n) == (34 * n, 30 * n, 30)
    assert bench.algorithmic_bytes('c3', n) == (46 * n, 28 * n, 28)
    assert bench.algorithmic_bytes('c2r', 443_357_184) == (34 * 443_357_184, 30 * 443_357_184, 30)


def test_committed_traffic_summaries_parse():
    """Every committed counter summary states what it counts (L2 -> fabric requests), the bytes the MALL serves by
    design, and measured / algorithmic bytes consistent with its own fields."""
    n = 430_662_912
    alg = {('adam_cast', 'c2'): 30 * n, ('adam_cast', 'c3'): 28 * n, ('sumsq', 'c2'): 4 * n,
           ('owner_sum', 'c3'): 18 * n, ('adam_cast', 'dropin'): 32 * n}
    for (kernel, workload), bytes_ in alg.items():
        t = bench.load_traffic(kernel, workload)
        assert t is not None, (kernel, workload)
        assert 'MALL' in t['counted_at'] and t['mall_served_bytes_by_design'] >= 0
        total = t['l2_to_fabric_read_bytes'] + t['l2_to_fabric_write_bytes']
        assert total == t['l2_to_fabric_bytes_per_launch']
        assert t['algorithmic_read_bytes'] + t['algorithmic_write_bytes'] == bytes_
        assert abs(total / bytes_ - t['measured_over_algorithmic']) < 1e-4
        assert 1.0 <= t['measured_over_algorithmic'] < 1.01, (kernel, workload)
        assert t['dram_bytes_per_launch_estimate'] == total - t['mall_served_bytes_by_design']


def test_config_sizes(pkg):
    """Parameter and tensor counts of every workload: C2 = C4 / 8; C2R is the largest owner of YOCO-3B's greedy
    8-rank partition; C4R is the whole 240-tensor model."""
    from faster_yoco_amd import configs, layout
    import math
    want = {'c1': (9_438_208, 4), 'c2': (430_662_912, 38), 'c3': (430_662_912, 38), 'c5': (430_662_912, 38),
            'c4': (3_445_303_296, 304), 'c2r': (443_357_184, 9), 'c4r': (3_445_303_296, 240)}
    for name, (n, t) in want.items():
        assert (configs.numel(name), len(configs.shapes(name))) == (n, t), name
    _, sizes = layout.greedy_partition([math.prod(s) for s in configs.shapes('c4r')], 8)
    assert max(sizes) == configs.numel('c2r') and sizes.index(max(sizes)) == 0
