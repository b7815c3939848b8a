"""ctypes binding of libnpu_host.so (include/npu_cost.h): the cost model, the
split rules and the MI355X target, over graphs built from parsed functions."""
from __future__ import annotations

import ctypes as C
import os

from . import mlir
from ._lib import NpuLaunchPlan  # the struct only: does not load libnpu_amd.so

_HERE = os.path.dirname(os.path.abspath(__file__))
HOST_LIB_PATH = os.path.join(_HERE, "libnpu_host.so")

OP_KINDS = {
    "linalg.matmul": 0, "linalg.batch_matmul": 1, "linalg.conv_2d_nchw_fchw": 2,
    "linalg.conv_2d_nhwc_fhwc": 3, "linalg.depthwise_conv_2d_nhwc_hwc": 4,
    "linalg.generic": 5, "linalg.fill": 6, "linalg.transpose": 7, "tensor.pad": 8,
    "tensor.empty": 9, "arith.constant": 10, "func.return": 11,
    "tensor.collapse_shape": 12, "tensor.expand_shape": 13, "func.call": 14,
}
LINALG_KINDS = {0, 1, 2, 3, 4, 5, 6, 7}


class HWTarget(C.Structure):
    _fields_ = [
        ("num_cores", C.c_int64), ("sram_per_core", C.c_int64), ("dram_bandwidth", C.c_int64),
        ("sram_bandwidth", C.c_int64), ("matrix_throughput", C.c_int64),
        ("dsp_throughput", C.c_int64), ("dma_channels", C.c_int64),
        ("inter_core_sync_cost", C.c_int64), ("clock_ghz", C.c_double),
        ("interconnect", C.c_int32), ("reserved", C.c_int32), ("noc_bandwidth", C.c_int64),
        ("noc_latency_cycles", C.c_int64), ("shared_l1_size", C.c_int64),
    ]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_ if k != "reserved"}


class Roofline(C.Structure):
    _fields_ = [("flops", C.c_double), ("mem_bytes", C.c_double),
                ("arithmetic_intensity", C.c_double), ("time_sec", C.c_double),
                ("is_memory_bound", C.c_int32), ("reserved", C.c_int32),
                ("peak_attainable", C.c_double), ("efficiency", C.c_double)]


class ScheduleCost(C.Structure):
    _fields_ = [("compute_cycles", C.c_int64), ("dma_cycles", C.c_int64),
                ("total_cycles", C.c_int64), ("sram_peak_bytes", C.c_int64),
                ("num_tiles", C.c_int64), ("total_dma_bytes", C.c_int64),
                ("valid", C.c_int32), ("n_tile_sizes", C.c_int32), ("tile_sizes", C.c_int64 * 4)]

    @property
    def tiles(self):
        return [self.tile_sizes[i] for i in range(self.n_tile_sizes)]


class SpatialSplitCost(C.Structure):
    _fields_ = [("per_core_dma_in_bytes", C.c_int64), ("per_core_compute_cycles", C.c_int64),
                ("shared_data_bytes", C.c_int64), ("split_data_bytes", C.c_int64),
                ("halo_overhead_bytes", C.c_int64), ("needs_reduce", C.c_int32),
                ("reserved", C.c_int32), ("total_cycles", C.c_int64)]


class SubgraphCost(C.Structure):
    _fields_ = [(n, C.c_int64) for n in (
        "dma_in_cycles", "matrix_cycles", "dsp_cycles", "dma_out_cycles", "intermediate_dma",
        "pipelined_cycles", "unpipelined_cycles", "num_ops")]


class GpuParams(C.Structure):
    """npu_gpu_params: machine constants of the MI355X launch model."""

    _fields_ = [
        ("cus", C.c_int32), ("reserved", C.c_int32), ("clock_ghz", C.c_double),
        ("hbm_gbs", C.c_double), ("l2_bytes_per_clk_cu", C.c_double),
        ("lds_bytes_per_clk_cu", C.c_double), ("valu_instr_per_clk_cu", C.c_double),
        ("mfma_macs_per_clk_cu", C.c_double * 3), ("mem_latency_us", C.c_double),
        ("launch_us", C.c_double), ("wave_valu_clk", C.c_double),
        ("burst_bytes_per_clk_cu", C.c_double),
    ]


class LaunchCost(C.Structure):
    _fields_ = [
        ("time_us", C.c_double), ("hbm_us", C.c_double), ("cu_us", C.c_double),
        ("tile_compute_us", C.c_double), ("tile_xfer_us", C.c_double),
        ("tile_serial_us", C.c_double), ("tiles_per_cu", C.c_double),
        ("bound", C.c_int32), ("reserved", C.c_int32),
    ]


BOUNDS = ("hbm", "mfma", "lds", "valu", "l2", "latency")

_I32, _I64, _P = C.c_int32, C.c_int64, C.c_void_p
_PT = C.POINTER(HWTarget)
_PI32 = C.POINTER(C.c_int32)
_PI64 = C.POINTER(C.c_int64)

SIGNATURES = {
    "npu_hw_target_default": (None, [_PT]),
    "npu_hw_target_mi355x": (None, [_PT, _I32]),
    "npu_graph_create": (_P, []),
    "npu_graph_destroy": (None, [_P]),
    "npu_graph_add_value": (_I32, [_P, _PI64, _I32, _I32, _I32]),
    "npu_graph_add_op": (_I32, [_P, _I32, _PI32, _I32, _PI32, _I32, _I32, _PI32, _I32, _PI64, _I32]),
    "npu_graph_num_ops": (_I32, [_P]),
    "npu_host_last_error": (C.c_char_p, []),
    "npu_cm_op_macs": (_I64, [_P, _PT, _I32]),
    "npu_cm_compute_cycles": (_I64, [_P, _PT, _I32]),
    "npu_cm_dma_cycles": (_I64, [_PT, _I64]),
    "npu_cm_tensor_bytes": (_I64, [_PI64, _I32, _I32]),
    "npu_cm_roofline_raw": (_I32, [_PT, C.c_double, C.c_double, _I32, C.POINTER(Roofline)]),
    "npu_cm_roofline": (_I32, [_P, _PT, _PI32, _I32, C.POINTER(Roofline)]),
    "npu_cm_matmul_tile": (_I32, [_PT] + [_I64] * 8 + [C.POINTER(ScheduleCost)]),
    "npu_cm_conv2d_tile": (_I32, [_PT] + [_I64] * 15 + [C.POINTER(ScheduleCost)]),
    "npu_cm_tile_candidates": (_I32, [_I64, _PI64, _I32]),
    "npu_spec_reset": (_I32, []),
    "npu_cm_best_tile_config": (_I32, [_P, _PT, _I32, C.POINTER(ScheduleCost)]),
    "npu_cm_fusion_profitable": (_I32, [_P, _PT, _I32, _I32, _PI64]),
    "npu_cm_spatial_split": (_I32, [_P, _PT, _I32, _I32, _I64, C.POINTER(ScheduleCost)]),
    "npu_cm_spatial_split_detailed": (_I32, [_P, _PT, _I32, _I32, _I64,
                                             C.POINTER(SpatialSplitCost)]),
    "npu_cm_tile_alignment": (_I32, [_P, _PT, _PI32, _I32, _PI64]),
    "npu_cm_spill_strategy": (_I32, [_PT, _I64, _I64]),
    "npu_cm_subgraph": (_I32, [_P, _PT, _PI32, _I32, C.POINTER(SubgraphCost)]),
    "npu_cm_subgraph_fusion_profitable": (_I32, [_P, _PT, _PI32, _I32, _PI64]),
    "npu_spec_num_splits": (_I32, [_P, _I32]),
    "npu_spec_split": (_I32, [_P, _I32, _I32, _PI32, _PI32, _PI32]),
    "npu_spec_preferred_spatial_dim": (_I32, [_P, _I32]),
    "npu_gpu_params_mi355x": (None, [C.POINTER(GpuParams)]),
    "npu_cm_predict_launch": (_I32, [C.POINTER(NpuLaunchPlan), C.POINTER(GpuParams),
                                     C.POINTER(LaunchCost)]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(HOST_LIB_PATH):
            raise RuntimeError(f"libnpu_host.so not found at {HOST_LIB_PATH}: build it with make")
        h = C.CDLL(HOST_LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def _check(rc):
    if rc < 0:
        raise ValueError(lib().npu_host_last_error().decode())
    return rc


def default_target() -> HWTarget:
    t = HWTarget()
    lib().npu_hw_target_default(C.byref(t))
    return t


def target_from_params(params: dict) -> HWTarget:
    """The default target with a module's #npu.target parameters applied, as
    CostModelAnalysis does (lib/Analysis/CostModel.cpp:985-1000): the seven
    parameters replace the defaults, every other field keeps its default."""
    t = default_target()
    for k, v in params.items():
        setattr(t, k, int(v))
    return t


def mi355x_target(elem_bits=32) -> HWTarget:
    t = HWTarget()
    lib().npu_hw_target_mi355x(C.byref(t), elem_bits)
    return t


def _arr(ctype, xs):
    xs = list(xs)
    return (ctype * max(1, len(xs)))(*xs), len(xs)


class Graph:
    """A function body in the host library.  ``op_id[i]`` is the graph op of
    ``func.ops[i]``; ``value_id[name]`` the value of an SSA name."""

    def __init__(self, func: mlir.MFunc):
        self.func = func
        self.h = lib().npu_graph_create()
        self.value_id = {}
        self.op_id = []
        self.kinds = []
        for name, t in func.args:
            self._value(name, t)
        for op in func.ops:
            kind = OP_KINDS.get(op.name, 15)
            operands = [self._ref(n) for n in op.all_operands]
            results = [self._value(r, t) for r, t in zip(op.results, op.result_types)]
            iters = [0 if it == "parallel" else 1 for it in op.iterators]
            perm = op.attrs.get("permutation", [])
            a_ops, n_ops = _arr(C.c_int32, operands)
            a_res, n_res = _arr(C.c_int32, results)
            a_it, n_it = _arr(C.c_int32, iters)
            a_pm, n_pm = _arr(C.c_int64, perm)
            oid = _check(lib().npu_graph_add_op(self.h, kind, a_ops, n_ops, a_res, n_res,
                                                len(op.ins), a_it, n_it, a_pm, n_pm))
            self.op_id.append(oid)
            self.kinds.append(kind)

    def _value(self, name, t: mlir.TType):
        shape, rank = _arr(C.c_int64, t.shape)
        vid = _check(lib().npu_graph_add_value(self.h, shape, rank, t.bits, 1 if t.shaped else 0))
        self.value_id[name] = vid
        return vid

    def _ref(self, name):
        if name not in self.value_id:
            # an SSA name defined outside the subset (e.g. a block argument)
            self._value(name, mlir.TType([], "f32", shaped=False))
        return self.value_id[name]

    def linalg_ops(self):
        """Indices (into func.ops) of linalg ops, in block order."""
        return [i for i, k in enumerate(self.kinds) if k in LINALG_KINDS]

    def find(self, name_prefix, nth=0):
        idx = [i for i, op in enumerate(self.func.ops) if op.name.startswith(name_prefix)]
        return idx[nth]

    def __del__(self):
        try:
            lib().npu_graph_destroy(self.h)
        except Exception:
            pass


class CostModel:
    """Cost model queries on a Graph (op arguments are indices into func.ops)."""

    def __init__(self, graph: Graph, target: HWTarget):
        self.g = graph
        self.t = target

    def _op(self, i):
        return self.g.op_id[i]

    def op_macs(self, i):
        return _check(lib().npu_cm_op_macs(self.g.h, C.byref(self.t), self._op(i)))

    def compute_cycles(self, i):
        return _check(lib().npu_cm_compute_cycles(self.g.h, C.byref(self.t), self._op(i)))

    def dma_cycles(self, nbytes):
        return lib().npu_cm_dma_cycles(C.byref(self.t), nbytes)

    def roofline(self, ops):
        a, n = _arr(C.c_int32, [self._op(i) for i in ops])
        r = Roofline()
        _check(lib().npu_cm_roofline(self.g.h, C.byref(self.t), a, n, C.byref(r)))
        return r

    def best_tile_config(self, i):
        s = ScheduleCost()
        _check(lib().npu_cm_best_tile_config(self.g.h, C.byref(self.t), self._op(i), C.byref(s)))
        return s

    def fusion_profitable(self, producer, consumer):
        b = C.c_int64()
        f = _check(lib().npu_cm_fusion_profitable(self.g.h, C.byref(self.t), self._op(producer),
                                                  self._op(consumer), C.byref(b)))
        return bool(f), b.value

    def spatial_split(self, i, dim, chunks):
        s = ScheduleCost()
        _check(lib().npu_cm_spatial_split(self.g.h, C.byref(self.t), self._op(i), dim, chunks,
                                          C.byref(s)))
        return s

    def spatial_split_detailed(self, i, split_index, chunks):
        s = SpatialSplitCost()
        _check(lib().npu_cm_spatial_split_detailed(self.g.h, C.byref(self.t), self._op(i),
                                                   split_index, chunks, C.byref(s)))
        return s

    def tile_alignment(self, ops):
        a, n = _arr(C.c_int32, [self._op(i) for i in ops])
        o = C.c_int64()
        aligned = _check(lib().npu_cm_tile_alignment(self.g.h, C.byref(self.t), a, n, C.byref(o)))
        return bool(aligned), o.value

    def subgraph(self, ops):
        a, n = _arr(C.c_int32, [self._op(i) for i in ops])
        s = SubgraphCost()
        _check(lib().npu_cm_subgraph(self.g.h, C.byref(self.t), a, n, C.byref(s)))
        return s

    def subgraph_fusion_profitable(self, ops):
        a, n = _arr(C.c_int32, [self._op(i) for i in ops])
        b = C.c_int64()
        f = _check(lib().npu_cm_subgraph_fusion_profitable(self.g.h, C.byref(self.t), a, n,
                                                           C.byref(b)))
        return bool(f), b.value

    def spec_splits(self, i):
        n = _check(lib().npu_spec_num_splits(self.g.h, self._op(i)))
        out = []
        for k in range(n):
            od, it, par = C.c_int32(), C.c_int32(), C.c_int32()
            _check(lib().npu_spec_split(self.g.h, self._op(i), k, C.byref(od), C.byref(it),
                                        C.byref(par)))
            out.append((od.value, it.value, bool(par.value)))
        return out


def tile_candidates(dim):
    buf = (C.c_int64 * 64)()
    n = lib().npu_cm_tile_candidates(dim, buf, 64)
    return [buf[i] for i in range(min(n, 64))]


def spec_reset():
    """Forgets the conv tiling spec in force (built from the first conv asked
    about, as getTilingSpec's function-local static is once per npu-opt
    process): the next conv builds the next one."""
    lib().npu_spec_reset()


def matmul_tile(target, tm, tn, tk, M, N, K, dtype_bytes, extra=0):
    s = ScheduleCost()
    _check(lib().npu_cm_matmul_tile(C.byref(target), tm, tn, tk, M, N, K, dtype_bytes, extra,
                                     C.byref(s)))
    return s


def conv2d_tile(target, tn, tco, th, tw, N, Co, Ho, Wo, Ci, Kh, Kw, dtype_bytes, stride=(1, 1),
                extra=0):
    s = ScheduleCost()
    _check(lib().npu_cm_conv2d_tile(C.byref(target), tn, tco, th, tw, N, Co, Ho, Wo, Ci, Kh, Kw,
                                    stride[0], stride[1], dtype_bytes, extra, C.byref(s)))
    return s


def spill_strategy(target, working_set, intermediate_bytes):
    return "spill" if lib().npu_cm_spill_strategy(C.byref(target), working_set,
                                                 intermediate_bytes) else "retile"


# ---------------------------------------------------------------- pass decisions
class SpatialDecision(C.Structure):
    _fields_ = [("iter_dim", C.c_int32), ("out_dim", C.c_int32), ("dim_size", C.c_int64),
                ("tile_size", C.c_int64), ("full_iters", C.c_int64), ("peel_size", C.c_int64),
                ("cost", C.c_int64), ("n_candidates", C.c_int32), ("reserved", C.c_int32),
                ("cand_iter_dims", C.c_int32 * 8), ("cand_costs", C.c_int64 * 8)]

    @property
    def candidates(self):
        return [(self.cand_iter_dims[i], self.cand_costs[i]) for i in range(self.n_candidates)]


SIGNATURES.update({
    "npu_pass_fusion_groups": (_I32, [_P, _PT, _PI32, _I32, _PI32, _I32]),
    "npu_pass_tile_and_fuse": (_I32, [_P, _PT, _I32, C.POINTER(ScheduleCost)]),
    "npu_pass_outline_groups": (_I32, [_P, _PT, _PI32, _I32, _PI32, _I32]),
    "npu_pass_outline_group_info": (_I32, [_P, _PT, _I32, C.c_char_p, _I32, _PI32, _PI32, _PI32,
                                           _PI32, _I32]),
    "npu_pass_spatial": (_I32, [_P, _PT, _I32, _I64, C.POINTER(SpatialDecision)]),
    "npu_pass_temporal": (_I32, [_P, _PT, _I32, C.POINTER(ScheduleCost), _PI64, _I32]),
})


def _groups(fn, g: Graph, t: HWTarget):
    ops = (C.c_int32 * 4096)()
    sizes = (C.c_int32 * 1024)()
    n = _check(fn(g.h, C.byref(t), ops, 4096, sizes, 1024))
    inv = {oid: i for i, oid in enumerate(g.op_id)}
    out, k = [], 0
    for i in range(n):
        out.append([inv[ops[k + j]] for j in range(sizes[i])])
        k += sizes[i]
    return out


def fusion_groups(g: Graph, t: HWTarget):
    """npu-fusion groups, as lists of indices into func.ops."""
    return _groups(lib().npu_pass_fusion_groups, g, t)


def tile_and_fuse(g: Graph, t: HWTarget, consumer):
    s = ScheduleCost()
    tiled = _check(lib().npu_pass_tile_and_fuse(g.h, C.byref(t), g.op_id[consumer], C.byref(s)))
    return bool(tiled), s


def outline_groups(g: Graph, t: HWTarget):
    """npu-outline-fused-groups: [{ops, name, inputs, outputs}] with SSA names."""
    groups = _groups(lib().npu_pass_outline_groups, g, t)
    names = {v: k for k, v in g.value_id.items()}
    out = []
    for i, ops in enumerate(groups):
        buf = C.create_string_buffer(512)
        ins, outs = (C.c_int32 * 64)(), (C.c_int32 * 64)()
        ni, no = C.c_int32(), C.c_int32()
        _check(lib().npu_pass_outline_group_info(g.h, C.byref(t), i, buf, 512, ins, C.byref(ni),
                                                 outs, C.byref(no), 64))
        out.append({"ops": ops, "name": buf.value.decode(),
                    "inputs": [names[ins[j]] for j in range(ni.value)],
                    "outputs": [names[outs[j]] for j in range(no.value)]})
    return out


def spatial(g: Graph, t: HWTarget, op, cores):
    d = SpatialDecision()
    tiled = _check(lib().npu_pass_spatial(g.h, C.byref(t), g.op_id[op], cores, C.byref(d)))
    return d if tiled else None


def temporal(g: Graph, t: HWTarget, op):
    s = ScheduleCost()
    ts = (C.c_int64 * 16)()
    n = _check(lib().npu_pass_temporal(g.h, C.byref(t), g.op_id[op], C.byref(s), ts, 16))
    return (list(ts[:n]), s) if n else (None, None)


# ---------------------------------------------------------------- buffers after tiling
ROLES = ("input", "output", "intermediate")


class SramBuffer(C.Structure):
    _fields_ = [("value", C.c_int32), ("role", C.c_int32), ("bytes", C.c_int64),
                ("first_use", C.c_int64), ("last_use", C.c_int64), ("in_loop", C.c_int32),
                ("double_buffered", C.c_int32), ("addr", C.c_int64), ("addr_pong", C.c_int64),
                ("prefetch_addr", C.c_int64), ("spilled", C.c_int32), ("reserved", C.c_int32)]


class SramSummary(C.Structure):
    _fields_ = [("spilled", C.c_int64), ("prefetched", C.c_int64), ("prefetch_bytes", C.c_int64),
                ("peak_bytes", C.c_int64), ("free_after", C.c_int64)]


class KernelCost(C.Structure):
    _fields_ = [("flops", C.c_double), ("mem_bytes", C.c_double),
                ("arithmetic_intensity", C.c_double), ("time_sec", C.c_double),
                ("efficiency", C.c_double), ("memory_bound", C.c_int32), ("reserved", C.c_int32),
                ("dma_in_bytes", C.c_int64), ("dma_out_bytes", C.c_int64),
                ("matrix_cycles", C.c_int64), ("dsp_cycles", C.c_int64),
                ("peak_sram_bytes", C.c_int64), ("num_tile_iterations", C.c_int64),
                ("num_linalg_ops", C.c_int64), ("sram_budget", C.c_int64)]


SIGNATURES.update({
    "npu_pass_bufferize": (_I32, [_P, _PI32, _I32, _PI64, _I32, C.POINTER(SramBuffer), _I32]),
    "npu_pass_sram_allocation": (_I32, [C.POINTER(SramBuffer), _I32, _I64, C.POINTER(SramSummary)]),
    "npu_pass_barrier_alloc": (_I32, [_PI32, _I32, _I64, _PI64, _PI64, _PI64]),
    "npu_pass_cost_evaluate": (_I32, [_P, _PT, _PI32, _I32, C.POINTER(SramBuffer), _I32, _I64,
                                      C.POINTER(KernelCost)]),
})


def bufferize(g: Graph, ops, tile_bytes=None):
    """npu-bufferize's DMA insertion for the tile loop whose body is `ops`
    (indices into func.ops): one SRAM buffer per shaped operand defined
    outside, with its role and liveness.  `tile_bytes` maps SSA names to the
    bytes of their tile slice (else the full tensor)."""
    a_ops, n_ops = _arr(C.c_int32, [g.op_id[i] for i in ops])
    by = None
    nb = 0
    if tile_bytes:
        nb = max(g.value_id.values()) + 1
        by = (C.c_int64 * nb)()
        for name, b in tile_bytes.items():
            by[g.value_id[name]] = b
    n = _check(lib().npu_pass_bufferize(g.h, a_ops, n_ops, by, nb, None, 0))
    out = (SramBuffer * max(n, 1))()
    lib().npu_pass_bufferize(g.h, a_ops, n_ops, by, nb, out, n)
    return list(out[:n])


def sram_allocation(buffers, sram_size):
    """npu-sram-allocation's dual-end plan of `buffers` (SramBuffer list, planned
    in place) for an SRAM of `sram_size` bytes; returns the summary."""
    arr = (SramBuffer * max(len(buffers), 1))(*buffers)
    summ = SramSummary()
    _check(lib().npu_pass_sram_allocation(arr, len(buffers), sram_size, C.byref(summ)))
    for i in range(len(buffers)):
        buffers[i] = arr[i]
    return summ


def cost_evaluate(g: Graph, t: HWTarget, ops, buffers, tile_iterations=1) -> KernelCost:
    a_ops, n_ops = _arr(C.c_int32, [g.op_id[i] for i in ops])
    arr = (SramBuffer * max(len(buffers), 1))(*buffers)
    kc = KernelCost()
    _check(lib().npu_pass_cost_evaluate(g.h, C.byref(t), a_ops, n_ops, arr, len(buffers),
                                        tile_iterations, C.byref(kc)))
    return kc


def cost_json(name, kc: KernelCost, extra=None) -> str:
    """The COST_JSON line of CostEvaluatePass.cpp:135-158 (same keys, same
    order), optionally followed by extra keys (the MI355X prediction)."""
    import json
    rec = {"name": name, "flops": kc.flops, "mem_bytes": kc.mem_bytes,
           "arithmetic_intensity": kc.arithmetic_intensity, "time_sec": kc.time_sec,
           "is_memory_bound": bool(kc.memory_bound), "efficiency": kc.efficiency,
           "dma_in_bytes": kc.dma_in_bytes, "dma_out_bytes": kc.dma_out_bytes,
           "matrix_cycles": kc.matrix_cycles, "dsp_cycles": kc.dsp_cycles,
           "peak_sram_bytes": kc.peak_sram_bytes, "num_tile_iterations": kc.num_tile_iterations,
           "num_linalg_ops": kc.num_linalg_ops, "sram_budget": kc.sram_budget,
           "bottleneck": "memory" if kc.memory_bound else "compute"}
    if extra:
        rec.update(extra)
    return "COST_JSON: " + json.dumps(rec)


def mi355x_gpu() -> GpuParams:
    """The calibrated MI355X constants of the launch model."""
    g = GpuParams()
    lib().npu_gpu_params_mi355x(C.byref(g))
    return g


def predict_launch(plan: NpuLaunchPlan, gpu: GpuParams = None) -> LaunchCost:
    """Launch-model time of one kernel launch (npu_cm_predict_launch)."""
    out = LaunchCost()
    _check(lib().npu_cm_predict_launch(C.byref(plan), C.byref(gpu or mi355x_gpu()), C.byref(out)))
    return out


def predict_block(plans, gpu: GpuParams = None):
    """Predicted time of a fused block: its launches back to back in a captured
    graph (each kernel's duration plus the per-launch cost).  Returns
    (total_us, [(kernel, LaunchCost), ...])."""
    gpu = gpu or mi355x_gpu()
    parts = [(p.kernel.decode(), predict_launch(p, gpu)) for p in plans]
    return sum(c.time_us + gpu.launch_us for _, c in parts), parts


# ---------------------------------------------------------------- barrier allocation
SCHED = {"dma_in": 0, "compute": 1, "dma_out": 2, "ignore": 3}


def barrier_alloc(kinds, pool=4):
    """npu-barrier-alloc (DMASchedulingPass.cpp:92-147) over ops given by their
    scheduling class in program order ('dma_in', 'compute', 'dma_out',
    'ignore'): per op (subgraph, barrier_id, generation), -1 for ignored."""
    n = len(kinds)
    k = (C.c_int32 * max(n, 1))(*[SCHED[x] for x in kinds])
    sg, bid, gen = ((C.c_int64 * max(n, 1))() for _ in range(3))
    _check(lib().npu_pass_barrier_alloc(k, n, int(pool), sg, bid, gen))
    return [(sg[i], bid[i], gen[i]) for i in range(n)]

