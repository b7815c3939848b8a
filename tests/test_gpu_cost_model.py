"""The launch model's per-kernel work terms against the hardware's counters.

Every entry point records launch plans whose vector-ALU terms (instructions
per tile besides the MFMAs, plus a persistent workgroup's one-time set-up)
are read from the kernels' compiled loop structure.  Here each configuration
runs once on the GPU, and each plan's vector instructions per wave

    (tile_valu * tiles + wg_setup_valu * grid) / (unit_waves * grid)

(tile_valu and wg_setup_valu summed over a grid unit's waves) are compared with what the counters measured for
the same kernel: (SQ_INSTS_VALU - SQ_INSTS_MFMA) / SQ_WAVES in
profiles/mfma_lds_counters_all_configs.txt (the file's valu/wv column),
within 15 %.
"""
import os
import re

import pytest
import torch

from npu_amd import configs, groups

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROFILE = os.path.join(ROOT, "profiles", "mfma_lds_counters_all_configs.txt")
TOL = 0.15


def counters():
    """workload -> [(kernel, valu per wave)] in launch order."""
    rows = {}
    with open(PROFILE) as f:
        for ln in f:
            m = re.match(r"^(\S+)\s+(.+?)\s+(\d+)\s+(\d+)\s+([\d.]+)\s+([\d.]+)\s+(\d+)\s+(\d+)"
                         r"\s+(\d+)\s+(\d+)\s*$", ln)
            if m and not ln.startswith("#"):
                rows.setdefault(m.group(1), []).append((m.group(2).strip(), int(m.group(7))))
    return rows


def predicted_valu_per_wave(p):
    waves = (p.unit_waves or 4) * float(p.grid)
    return (p.tile_valu * p.tiles + p.wg_setup_valu * p.grid) / waves


@pytest.mark.parametrize("w", configs.all_workloads(), ids=lambda w: w.name)
def test_plan_vector_instructions_match_the_counters(cuda, w):
    table = counters()
    assert w.name in table, f"{w.name}: no counter row in {PROFILE}"
    d = configs.to_device(w.make_inputs())
    o = w.make_outputs(d)
    print(f"plans of {w.name}", flush=True)
    with groups.collect_plans() as cp:
        w.run(d, o, None)
    torch.cuda.synchronize()
    rows = table[w.name]
    assert len(cp.plans) == len(rows), (w.name, [p.kernel for p in cp.plans], rows)
    errs = []
    for p, (kernel, measured) in zip(cp.plans, rows):
        if p.kernel == b"llama_causal_attention":
            # its plan is its busiest workgroup's (the last query block's key
            # walk, what bounds the launch's time); the counters average
            # every workgroup, most of which walk fewer key blocks
            assert predicted_valu_per_wave(p) >= measured
            continue
        pred = predicted_valu_per_wave(p)
        err = pred / measured - 1.0
        print(f"  {p.kernel.decode():32s} predicted {pred:8.1f}  measured {measured:6d}  "
              f"({err:+.1%})", flush=True)
        errs.append((kernel, pred, measured, err))
    bad = [e for e in errs if abs(e[3]) > TOL]
    assert not bad, f"{w.name}: {bad}"
