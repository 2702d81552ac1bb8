"""Python binding of libsplash_q4.so (include/splash_q4.h) for tests, benchmarks and scripting.

The library is the product: every call here goes through its C ABI. Device memory comes from torch (tensors are
passed as {data_ptr, bytes} views) and launches go on torch's current HIP stream. Loading fails loudly when the
library is missing: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
from ctypes import POINTER, Structure, byref, c_char_p, c_int, c_uint32, c_uint64, c_void_p

PACKAGE_ROOT = pathlib.Path(__file__).resolve().parent.parent
LIBRARY = PACKAGE_ROOT / "lib" / "libsplash_q4.so"
HEADER = PACKAGE_ROOT.parent / "include" / "splash_q4.h"

SQ_OK, SQ_INVALID_ARGUMENT, SQ_RUNTIME_ERROR = 0, 1, 2
FMT_Q4K, FMT_AF4G32, FMT_AF4G64, FMT_AF4G128 = 0, 25, 26, 27
FMT_Q5K, FMT_Q6K, FMT_Q80, FMT_AF8G64 = 3, 4, 6, 35
PHASE_PREFILL, PHASE_DECODE = 0, 1
EPILOGUE_NONE, EPILOGUE_RESIDUAL, EPILOGUE_GATE_UP, EPILOGUE_UP_WITH_GATE = 0, 1, 2, 3
TILE_STAGED, TILE_PREFILL, TILE_REGISTER = 0, 1, 2
OUTPUT_BF16, OUTPUT_F32 = 0, 1
FMT_BF16, FLOAT32_ROWS = 41, 0xFFFFFFFF
LINEAR_INPUT_PLAIN, LINEAR_INPUT_TABLE16, LINEAR_INPUT_HALF_ROWS = 0, 1, 2

# (block_elements, block_bytes, plane0_bytes, meta_bytes, meta_groups, plane1_bytes) of QuantFormat.h:159-192.
FORMATS = {
    FMT_Q4K: (256, 144, 16, 16, 8, 0),
    FMT_Q5K: (256, 176, 16, 16, 8, 4),
    FMT_Q6K: (256, 210, 16, 20, 8, 8),
    FMT_Q80: (32, 34, 32, 2, 1, 0),
    FMT_AF4G32: (32, 20, 16, 4, 1, 0),
    FMT_AF4G64: (64, 36, 16, 4, 2, 0),
    FMT_AF4G128: (128, 68, 16, 4, 4, 0),
    FMT_AF8G64: (64, 68, 32, 4, 2, 0),
}


class Buffer(Structure):
    _fields_ = [("ptr", c_void_p), ("bytes", c_uint64)]


class Segment(Structure):
    _fields_ = [("plane0", Buffer), ("plane1", Buffer), ("meta", Buffer), ("output_size", c_uint32),
                ("input_size", c_uint32), ("column_offset", c_uint32), ("format_id", c_uint32)]


class Projection(Structure):
    _fields_ = [("output_size", c_uint32), ("input_size", c_uint32), ("segment_count", c_uint32),
                ("destination", c_uint32), ("segments", Segment * 3)]


class LinearWorkload(Structure):
    _fields_ = [("output_size", c_uint32), ("input_size", c_uint32), ("rows", c_uint32), ("phase", c_uint32),
                ("epilogue", c_uint32)]


class LinearConfig(Structure):
    _fields_ = [("tile", c_uint32), ("splits", c_uint32), ("spread", c_uint32), ("one_gate_up_pass", c_uint32),
                ("sixteen_rows", c_uint32)]


class LinearPlan(Structure):
    _fields_ = [("workload", LinearWorkload), ("config", LinearConfig), ("destination", c_uint32),
                ("storage_rows", c_uint32)]


class LinearScratchSize(Structure):
    _fields_ = [(n, c_uint64) for n in ("input", "sums", "partials", "counters", "rotated")]


class LinearScratch(Structure):
    _fields_ = [(n, Buffer) for n in ("input", "sums", "partials", "counters", "rotated")]


class PreparedInput(Structure):
    _fields_ = [("source", Buffer), ("layout", c_uint32)]


class LinearBuffers(Structure):
    _fields_ = [("input", Buffer), ("output", Buffer), ("residual", Buffer), ("gate_scratch", Buffer),
                ("scratch", LinearScratch), ("prepared", PreparedInput)]


class NormWeights(Structure):
    _fields_ = [("buffer", Buffer), ("float32", c_uint32)]


class Device(Structure):
    _fields_ = [("compute_units", c_uint32)]


ROUTER_SOFTMAX, ROUTER_SIGMOID_NORMALIZED = 0, 1


class MoeShape(Structure):
    _fields_ = [(n, c_uint32) for n in ("hidden_size", "experts", "experts_per_token", "expert_intermediate_size",
                                        "expert_format", "router", "shared_slices", "shared_gated")]


_MOE_WORKSPACE = ("selected_experts", "routing_weights", "tile_descriptors", "tile_count", "grouped_routes",
                  "route_rows", "grouped_input", "expert_intermediate", "expert_output")


class MoeWorkspace(Structure):
    _fields_ = [(n, c_uint64) for n in _MOE_WORKSPACE]


MOE_EXPERT_TILE_M8, MOE_EXPERT_TILE_M32 = 8, 32
MOE_GGUF_TILE_STAGED, MOE_GGUF_TILE_REGISTER = 0, 1
FLOAT_TILE_SIMDGROUP, FLOAT_TILE_NEURAL_ACCELERATOR = 0, 1


class MoeConfig(Structure):
    _fields_ = [(n, c_uint32) for n in ("expert_tile", "gguf_tile", "router_tile", "cpu_bf16_experts")]


class MoePlan(Structure):
    _fields_ = [("shape", MoeShape), ("rows", c_uint32), ("phase", c_uint32), ("tile_rows", c_uint32),
                ("maximum_tiles", c_uint32), ("config", MoeConfig), ("workspace", MoeWorkspace)]


class MoeWeights(Structure):
    _fields_ = [("gate", Segment), ("up", Segment), ("down", Segment), ("slot_table", Buffer), ("slots", c_uint32),
                ("shared_gate", Segment), ("shared_up", Segment), ("shared_down", Segment),
                ("shared_scalar_gate", Buffer), ("router", Segment)]


class ExpertLoadProjection(Structure):
    _fields_ = [("format_id", c_uint32), ("rows", c_uint32), ("columns", c_uint32), ("row_bytes", c_uint32),
                ("planes", c_uint64 * 3), ("slot_bytes", c_uint64 * 3)]


class ExpertLoadParams(Structure):
    _fields_ = [("projections", ExpertLoadProjection * 3)]


class MoeScratch(Structure):
    _fields_ = [(n, Buffer) for n in _MOE_WORKSPACE]


class MoeBuffers(Structure):
    _fields_ = [("input", Buffer), ("residual", Buffer), ("output", Buffer), ("scratch", MoeScratch),
                ("verify_rows", Buffer)]


class SqError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class InvalidArgument(SqError, ValueError):
    pass


_lib = None

# name -> argtypes, for every entry point of include/splash_q4.h.
_SIGNATURES = {
    "sq_last_error": [],
    "sq_version": [],
    "sq_linear_plan_for": [POINTER(Device), POINTER(LinearWorkload), POINTER(Projection), POINTER(Projection),
                           POINTER(LinearPlan)],
    "sq_linear_plan_config": [POINTER(LinearWorkload), POINTER(LinearConfig), c_uint32, POINTER(LinearPlan)],
    "sq_linear_decode_plan": [POINTER(Device), POINTER(Projection), c_uint32, c_uint32, POINTER(Projection),
                              POINTER(LinearPlan)],
    "sq_linear_prefill_plan": [POINTER(Device), POINTER(Projection), c_uint32, c_uint32, POINTER(LinearPlan)],
    "sq_linear_plan_scratch": [POINTER(LinearPlan), POINTER(LinearScratchSize), POINTER(c_uint64)],
    "sq_linear_decode_scratch_size": [POINTER(Device), c_uint32, c_uint32, POINTER(LinearScratchSize)],
    "sq_linear_prefill_scratch_size": [POINTER(Device), c_uint32, c_uint32, POINTER(LinearScratchSize)],
    "sq_require_segment_planes": [POINTER(Segment), c_char_p, c_uint32],
    "sq_linear_add": [c_void_p, POINTER(LinearBuffers), POINTER(Projection), POINTER(LinearPlan), POINTER(Projection)],
    "sq_linear_add_prepared": [c_void_p, POINTER(LinearBuffers), POINTER(Projection), POINTER(LinearPlan),
                               POINTER(Projection), POINTER(PreparedInput)],
    "sq_linear_plan_input": [POINTER(LinearPlan), POINTER(c_uint32)],
    "sq_linear_add_static": [c_void_p, POINTER(LinearBuffers), POINTER(Projection), POINTER(LinearPlan),
                             POINTER(Projection)],
    "sq_norm_add_rms": [c_void_p, Buffer, POINTER(NormWeights), Buffer, c_uint32, c_uint32, POINTER(LinearScratch),
                        c_uint32, POINTER(PreparedInput)],
    "sq_float_add": [c_void_p, Buffer, POINTER(Segment), Buffer, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32],
    "sq_linear_float_tile": [POINTER(Device), c_uint32, c_uint32, c_uint32, POINTER(c_uint32)],
    "sq_linear_decode_storage_rows": [POINTER(Device), c_uint32, c_uint32, c_uint32, POINTER(c_uint32)],
    "sq_linear_add_prefill": [POINTER(Device), c_void_p, Buffer, POINTER(Projection), Buffer, c_uint32,
                              POINTER(LinearScratch)],
    "sq_linear_add_prefill_residual": [POINTER(Device), c_void_p, Buffer, POINTER(Projection), Buffer, Buffer,
                                       c_uint32, POINTER(LinearScratch)],
    "sq_linear_add_prefill_up_with_gate": [POINTER(Device), c_void_p, Buffer, POINTER(Projection), Buffer, Buffer,
                                           c_uint32, POINTER(LinearScratch)],
    "sq_linear_add_prefill_swiglu": [POINTER(Device), c_void_p, POINTER(Projection), POINTER(Projection),
                                     POINTER(Projection), Buffer, Buffer, Buffer, POINTER(LinearScratch), Buffer,
                                     Buffer, c_uint32],
    "sq_gguf_repack": [c_void_p, Buffer, Buffer, c_void_p],
    "sq_mlx_repack": [c_void_p, c_uint32, c_uint32, c_uint32, Buffer, Buffer, Buffer, Buffer, Buffer],
    "sq_dequant": [c_void_p, POINTER(Segment), Buffer, Buffer],
    "sq_diag_stream_read": [c_void_p, Buffer, Buffer, c_uint32, c_uint32],
    "sq_diag_mfma_peak": [c_void_p, Buffer, c_uint32, c_uint32, c_uint32],
    "sq_moe_config_for": [POINTER(MoeShape), c_uint32, c_uint32, POINTER(MoeConfig)],
    "sq_moe_prefill_plan": [POINTER(MoeShape), c_uint32, POINTER(MoeConfig), POINTER(MoePlan)],
    "sq_moe_decode_plan": [POINTER(MoeShape), c_uint32, POINTER(MoeConfig), POINTER(MoePlan)],
    "sq_moe_decode_rows_plan": [POINTER(MoeShape), c_uint32, POINTER(MoePlan)],
    "sq_moe_router_width": [POINTER(MoeShape)],
    "sq_moe_add": [c_void_p, POINTER(MoeBuffers), POINTER(MoeWeights), POINTER(MoePlan)],
    "sq_moe_add_routing": [c_void_p, POINTER(MoeBuffers), POINTER(MoeWeights), POINTER(MoePlan)],
    "sq_moe_add_routed": [c_void_p, POINTER(MoeBuffers), POINTER(MoeWeights), POINTER(MoePlan)],
    "sq_moe_add_routes": [c_void_p, Buffer, POINTER(Segment), Buffer, Buffer, Buffer, Buffer, c_uint32,
                          POINTER(MoeShape), c_uint32],
    "sq_moe_expert_load": [c_void_p, Buffer, Buffer, Buffer, Buffer, POINTER(ExpertLoadParams), c_uint32, Buffer],
    "sq_moe_expert_load_groups": [POINTER(ExpertLoadParams)],
}


def lib() -> ctypes.CDLL:
    """The loaded library; raises when it has not been built."""
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            raise RuntimeError(f"{LIBRARY} is not built: run __graft_entry__.build() (make -C splash-desktop_amd)")
        handle = ctypes.CDLL(str(LIBRARY))
        for name, args in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = (c_char_p if name in ("sq_last_error", "sq_version") else
                          c_uint32 if name in ("sq_moe_router_width", "sq_moe_expert_load_groups") else c_int)
        _lib = handle
    return _lib


def call(name: str, *args) -> None:
    code = getattr(lib(), name)(*args)
    if code != SQ_OK:
        message = lib().sq_last_error().decode()
        raise (InvalidArgument if code == SQ_INVALID_ARGUMENT else SqError)(code, message)


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


# ---------------------------------------------------------------- buffers and weights

def view(tensor=None, nbytes: int | None = None) -> Buffer:
    """A {ptr, bytes} view of a torch tensor (or a null view)."""
    if tensor is None:
        return Buffer(None, 0)
    total = tensor.numel() * tensor.element_size()
    return Buffer(tensor.data_ptr(), total if nbytes is None else nbytes)


def stream_handle():
    import torch
    return c_void_p(torch.cuda.current_stream().cuda_stream)


def plane_bytes(fmt: int, n: int, k: int) -> tuple[int, int]:
    """Bytes of plane0 and meta for an n x k tensor."""
    _, _, p0, meta_bytes, meta_groups, _ = FORMATS[fmt]
    groups = k // 32
    return n * groups * p0, n * (groups // meta_groups) * meta_bytes


def segment(fmt: int, n: int, k: int, plane0, meta, column_offset: int = 0, plane1=None) -> Segment:
    return Segment(view(plane0), view(plane1), view(meta), n, k, column_offset, fmt)


def projection(segments, output_size: int | None = None, destination: int = OUTPUT_BF16) -> Projection:
    if isinstance(segments, Segment):
        segments = [segments]
    p = Projection()
    p.output_size = output_size if output_size is not None else sum(s.output_size for s in segments)
    p.input_size = segments[0].input_size
    p.segment_count = len(segments)
    p.destination = destination
    for i, s in enumerate(segments):
        p.segments[i] = s
    return p


def device(compute_units: int = 0) -> Device:
    return Device(compute_units)


# ---------------------------------------------------------------- planning

def plan_for(workload: LinearWorkload, proj: Projection | None = None, gate: Projection | None = None,
             dev: Device | None = None) -> LinearPlan:
    out = LinearPlan()
    call("sq_linear_plan_for", byref(dev or Device(0)), byref(workload), byref(proj) if proj else None,
         byref(gate) if gate else None, byref(out))
    return out


def plan_config(workload: LinearWorkload, config: LinearConfig, destination: int = OUTPUT_BF16) -> LinearPlan:
    out = LinearPlan()
    call("sq_linear_plan_config", byref(workload), byref(config), destination, byref(out))
    return out


def decode_workload(n: int, k: int, rows: int, epilogue: int = EPILOGUE_NONE) -> LinearWorkload:
    return LinearWorkload(n, k, rows, PHASE_DECODE, epilogue)


def prefill_workload(n: int, k: int, rows: int, epilogue: int = EPILOGUE_NONE) -> LinearWorkload:
    return LinearWorkload(n, k, rows, PHASE_PREFILL, epilogue)


def scratch_size(plan: LinearPlan) -> tuple[LinearScratchSize, int]:
    size, gate = LinearScratchSize(), c_uint64(0)
    call("sq_linear_plan_scratch", byref(plan), byref(size), byref(gate))
    return size, gate.value


class Scratch:
    """Device scratch for a plan (zeroed at allocation, as the counters require)."""

    def __init__(self, plan: LinearPlan, device_name: str = "cuda"):
        import torch
        size, gate = scratch_size(plan)
        alloc = lambda b: torch.zeros(max(int(b), 0) // 4 + 1, dtype=torch.int32, device=device_name) if b else None
        self.input, self.sums = alloc(size.input), alloc(size.sums)
        self.partials, self.counters = alloc(size.partials), alloc(size.counters)
        self.gate = torch.zeros(gate // 2 + 1, dtype=torch.int16, device=device_name) if gate else None

    def struct(self) -> LinearScratch:
        return LinearScratch(view(self.input), view(self.sums), view(self.partials), view(self.counters), view(None))


def linear_add(plan: LinearPlan, proj: Projection, input, output, residual=None, gate_scratch=None,
               scratch: LinearScratch | None = None, gate: Projection | None = None, stream=None) -> None:
    buffers = LinearBuffers(view(input), view(output), view(residual), view(gate_scratch),
                            scratch if scratch is not None else LinearScratch())
    call("sq_linear_add", stream if stream is not None else stream_handle(), byref(buffers), byref(proj),
         byref(plan), byref(gate) if gate else None)


def mlx_repack(fmt: int, rows: int, k: int, weight, scales, biases, plane0, meta, stream=None) -> None:
    call("sq_mlx_repack", stream if stream is not None else stream_handle(), fmt, rows, k, view(weight), view(scales),
         view(biases), view(plane0), view(meta))


def gguf_repack(src, dst, rows: int, k: int, fmt: int, src_row_bytes: int, dst_meta: int, stream=None,
                dst_plane1: int = 0) -> None:
    params = (c_uint32 * 6)(rows, k, fmt, src_row_bytes, dst_plane1, dst_meta)
    call("sq_gguf_repack", stream if stream is not None else stream_handle(), view(src), view(dst), params)


def dequant(seg: Segment, values=None, halves=None, stream=None) -> None:
    call("sq_dequant", stream if stream is not None else stream_handle(), byref(seg), view(values), view(halves))


def stream_read(src, sink, workgroups: int, threads: int, nbytes: int | None = None, stream=None) -> None:
    """The read-only streaming kernel over `nbytes` of src (measurement aid, sq_diag_stream_read)."""
    call("sq_diag_stream_read", stream if stream is not None else stream_handle(), view(src, nbytes), view(sink),
         workgroups, threads)
