"""Post-pipeline modules on the GPU: the text npu-opt's passes produce (the
outlined @fused_* kernels, their tile-loop nests, the bufferized form with
npu.alloc_sram / npu.dma_copy), read back by npu_amd.reader and launched --
one launch per kernel's nest -- bit-identical to the lowering of the same
function before the passes (which the other GPU tests hold to the oracle),
and, for the reference's own workloads, within the f32 bound of the oracle.
"""
import numpy as np
import pytest
import torch

import refs
from npu_amd import blocks, configs, lower, npuopt, reader
from tolerance import RTOL_F32, check_bound

pytestmark = pytest.mark.gpu

FLAGS = {
    "pipeline": ["--npu-pipeline"],
    "mi355x": ["--npu-fusion", "--npu-outline-fused-groups", "--npu-spatial-tiling=num-cores=256",
               "--npu-core-mapping", "--npu-temporal-tiling=sram-size=163840", "--npu-bufferize",
               "--npu-sram-allocation=sram-size=163840", "--npu-barrier-alloc=barrier-pool-size=4",
               "--npu-cost-evaluate"],
}


def _module(text, flags):
    _, passes, _ = npuopt.parse_args(FLAGS[flags])
    mod, _, _ = npuopt.run_passes(text, passes)
    return mod


def _float_inputs(prog, seed):
    g = torch.Generator().manual_seed(seed)
    ins = {}
    for a, t in prog.func.args:
        x = torch.rand(t.shape, generator=g, dtype=torch.float32) * 2 - 1
        ins[a] = x.to(torch.bfloat16 if t.elem == "bf16" else torch.float32).cuda()
    return ins


def _same(a, b):
    ha, hb = configs.to_host(a), configs.to_host(b)
    return ha.shape == hb.shape and np.array_equal(ha.view(np.uint8), hb.view(np.uint8))


CASES = {
    "matmul_relu.mlir": lambda: blocks.reference_workload("matmul_relu.mlir"),
    "mlp.mlir": lambda: blocks.reference_workload("mlp.mlir"),
    "conv2d_relu.mlir": lambda: blocks.reference_workload("conv2d_relu.mlir"),
    "resnet_block.mlir": lambda: blocks.reference_workload("resnet_block.mlir"),
    "resnet50_block.mlir": lambda: blocks.reference_workload("resnet50_block.mlir"),
    "conv_bf16": lambda: blocks.conv_bias_act(2, 14, 14, 32, 64, elem="bf16"),
    "irb": lambda: blocks.inverted_residual(2, 16, 16, 24, 144),
}


@pytest.mark.parametrize("flags", list(FLAGS))
@pytest.mark.parametrize("name", list(CASES))
def test_post_pipeline_module_runs_like_its_source(cuda, name, flags):
    text = CASES[name]()
    print(f"post-pipeline module {name} [{flags}]", flush=True)
    direct = lower.lower_text(text)
    prog, flat = reader.lower_module(_module(text, flags))
    ins = _float_inputs(direct, 91)
    got = prog.run(ins)
    want = direct.run(ins)
    torch.cuda.synchronize()
    assert len(got) == len(want)
    for g, w in zip(got.values(), want.values()):
        assert _same(g, w), f"{name} [{flags}]: the module's launches differ from the source's"


def test_post_pipeline_matmul_relu_against_the_oracle(cuda):
    """test/matmul_relu.mlir after --npu-pipeline with the harness's fills
    0.01 (i + 1): the closed form 0.0512 (e2e_verify.py:288-309) and the
    oracle's loops."""
    prog, _ = reader.lower_module(_module(blocks.reference_workload("matmul_relu.mlir"),
                                          "pipeline"))
    ins = {a: torch.full(t.shape, 0.01 * (i + 1), dtype=torch.float32, device="cuda")
           for i, (a, t) in enumerate(prog.func.args)}
    (res,) = prog.run(ins).values()
    torch.cuda.synchronize()
    got = configs.to_host(res).astype(np.float64)
    assert np.all(np.abs(got - 0.0512) <= 1e-4 * 0.0512)
    A, B = (configs.to_host(ins[a]) for a, _ in prog.func.args)
    ref, mag = refs.matmul_bias_act(A, B, None, "relu")
    check_bound(configs.to_host(res), ref, mag, RTOL_F32, what="post-pipeline matmul_relu")


def test_post_pipeline_int8_bottleneck_is_bit_exact(cuda):
    w = configs.qbottleneck(1, H=14, W=14, C=64, M1=64)
    a = w.make_inputs()
    text = blocks.qbottleneck(1, 14, 14, 64, 64)
    ins = {k: configs.to_device({"x": v})["x"] for k, v in a.items()}
    ins["w1"] = ins["w1"].reshape(64, 1, 1, 64)
    ins["w3"] = ins["w3"].reshape(64, 1, 1, 64)
    direct = lower.lower_text(text)
    for flags in FLAGS:
        print(f"post-pipeline int8 bottleneck [{flags}]", flush=True)
        prog, _ = reader.lower_module(_module(text, flags))
        (got,) = prog.run(ins).values()
        (want,) = direct.run(ins).values()
        torch.cuda.synchronize()
        assert _same(got, want)
    ref = refs.qbottleneck(a)
    assert np.array_equal(configs.to_host(got), ref)


def test_post_pipeline_llama_layer(cuda):
    w = configs.llama_layer(S=64, D=128, H=2, F=192, seed=5)
    inp = w.make_inputs()
    d = configs.to_device(inp)
    d["cos"], d["sin"] = d.pop("cos_t"), d.pop("sin_t")
    text = blocks.llama_layer(64, 128, 2, 192)
    direct = lower.lower_text(text)
    want = direct.run(d)["%out"]
    for flags in FLAGS:
        print(f"post-pipeline llama layer [{flags}]", flush=True)
        prog, _ = reader.lower_module(_module(text, flags))
        assert len(prog.launches) == 5
        got = list(prog.run(d).values())[0]
        torch.cuda.synchronize()
        assert _same(got, want)


def test_ciface_compiled_caller_on_the_gpu(cuda):
    """tests/c/ciface_test: the compiled host side of matmul_relu.mlir after
    --npu-fusion --npu-outline-fused-groups, calling the generated
    _mlir_ciface_fused_fill_matmul_generic_0 once per 16-row tile on its
    subview descriptors: 0.0512 with the harness's fills, the oracle's
    loops within the f32 bound on seeded inputs."""
    import os
    import subprocess
    exe = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "tests", "c",
                       "ciface_test")
    print("ciface_test gpu", flush=True)
    p = subprocess.run([exe, "gpu"], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stdout + p.stderr
