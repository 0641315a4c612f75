"""ctypes binding of libtlm_hip.so (include/tlm_hip.h).

The library is the product: nothing in this package computes a result on the
CPU.  Importing fails with a clear error when the library has not been built
(``python -c "import __graft_entry__ as g; g.build()"``).
"""
import ctypes as C
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtlm_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"tierlm_amd: {LIB_PATH} is not built; run __graft_entry__.build() "
        "(hipcc --offload-arch=gfx950) first")

lib = C.CDLL(LIB_PATH)

vp, i32, i64, sz, f32 = C.c_void_p, C.c_int, C.c_int64, C.c_size_t, C.c_float


class Seg(C.Structure):
    """tlm_hip_seg"""
    _fields_ = [("dt", C.c_int32), ("packed", C.c_int32), ("W", vp), ("row_bytes", C.c_uint64),
                ("act", vp), ("y", vp), ("n", C.c_int64), ("rows", C.c_int64)]


class MoeDesc(C.Structure):
    """tlm_hip_moe_desc"""
    _fields_ = [("D", C.c_int64), ("de", C.c_int64), ("ds", C.c_int64),
                ("E", C.c_int32), ("k", C.c_int32), ("router", C.c_int32),
                ("routed_scale", C.c_float), ("eps", C.c_float),
                ("expert_dt", C.c_int32), ("shared_dt", C.c_int32),
                ("ffn_norm", vp), ("router_w", vp), ("router_bias", vp), ("mask", vp),
                ("experts", vp), ("sg", vp), ("su", vp), ("sd", vp), ("shared_gate_inp", vp)]


class ExpertSrc(C.Structure):
    """tlm_hip_expert_src"""
    _fields_ = [("layer", C.c_uint16), ("flags", C.c_uint16), ("id", C.c_uint32), ("dtype", C.c_int32),
                ("heat", C.c_float), ("seed", C.c_uint32), ("item_off", C.c_uint32 * 3),
                ("payload_len", C.c_uint64), ("payload", vp)]


FETCH = C.CFUNCTYPE(C.c_int, vp, C.c_int, C.c_int, vp, C.c_uint64)


class StoreOpts(C.Structure):
    """tlm_hip_store_opts"""
    _fields_ = [("d_model", C.c_int64), ("d_expert", C.c_int64), ("top_k", C.c_int32), ("prefetch", C.c_int32),
                ("pin_frac", C.c_double), ("budget_bytes", C.c_uint64), ("fetch", FETCH), ("fetch_user", vp)]


class ExpertRef(C.Structure):
    """tlm_hip_expert_ref"""
    _fields_ = [("slot", C.c_int32), ("mats", vp * 3)]


class StoreStats(C.Structure):
    """tlm_hip_store_stats"""
    _fields_ = [("hits", C.c_uint64), ("misses", C.c_uint64), ("prefetch_issued", C.c_uint64),
                ("prefetch_used", C.c_uint64), ("prefetch_dropped", C.c_uint64), ("bytes_read", C.c_uint64),
                ("evictions", C.c_uint64), ("wait_ns", C.c_uint64), ("slots", C.c_int32), ("pinned", C.c_int32),
                ("in_use", C.c_int32)]


class StackOpts(C.Structure):
    """tlm_hip_stack_opts"""
    _fields_ = [("lookahead", C.c_int32), ("lookahead_k", C.c_int32), ("interest", C.c_double),
                ("layer_heat", C.c_void_p), ("instinct", C.c_void_p), ("instinct_seen", C.c_void_p),
                ("host_routes", C.c_int32)]


class MoeHint(C.Structure):
    """tlm_hip_moe_hint"""
    _fields_ = [("desc", C.POINTER(MoeDesc)), ("layer", C.c_int32), ("workspace", vp)]


class PacketLoc(C.Structure):
    """tlm_hip_packet_loc"""
    _fields_ = [("type", C.c_uint16), ("layer", C.c_uint16), ("id", C.c_uint32), ("drive", C.c_uint8),
                ("replica_drive", C.c_uint8), ("flags", C.c_uint16), ("offset", C.c_uint64),
                ("replica_offset", C.c_uint64), ("total_len", C.c_uint64), ("crc32c", C.c_uint32),
                ("heat", C.c_float)]


class ModelGeom(C.Structure):
    """tlm_hip_model_geom"""
    _fields_ = [("arch", C.c_char * 32)] + [(n, C.c_uint32) for n in (
        "n_layers", "d_model", "n_heads", "n_kv_heads", "head_dim", "vocab", "n_experts", "top_k", "d_expert",
        "n_shared", "d_shared", "max_ctx", "router")] + [
        ("rope_theta", C.c_float), ("norm_eps", C.c_float), ("routed_scale", C.c_float),
        ("mtp_layers", C.c_uint32), ("rope_scale", C.c_uint32), ("rope_factor", C.c_float),
        ("rope_beta_fast", C.c_float), ("rope_beta_slow", C.c_float), ("rope_orig_len", C.c_uint32)]


class ModelSynthOpts(C.Structure):
    """tlm_hip_model_synth_opts"""
    _fields_ = [("expert_dt", C.c_int32), ("dense_dt", C.c_int32), ("qk_norm", C.c_int32), ("expert_pool", C.c_int32),
                ("seed", C.c_uint64), ("heat_gamma", C.c_double)]


class TensorRef(C.Structure):
    """tlm_hip_tensor_ref"""
    _fields_ = [("name", C.c_char * 48), ("dtype", C.c_uint32), ("ndim", C.c_uint32), ("shape", C.c_uint64 * 2),
                ("offset", C.c_uint64), ("nbytes", C.c_uint64)]


QDOT = C.CFUNCTYPE(C.c_float, vp, vp, C.c_int64, vp)
QMV = C.CFUNCTYPE(None, vp, C.c_size_t, vp, vp, C.c_int64, C.c_int64)


class QuantKernels(C.Structure):
    """tlm_hip_quant_kernels (layout of the reference's tlm_quant_kernels)."""
    _fields_ = [("name", C.c_char_p), ("dot", QDOT * 10), ("mv", QMV * 10)]


_SIGS = {
    "tlm_hip_init": (i32, [i32]),
    "tlm_hip_shutdown": (None, []),
    "tlm_hip_tier": (C.c_char_p, []),
    "tlm_hip_selftest_failures": (i32, []),
    "tlm_hip_errmsg": (C.c_char_p, []),
    "tlm_hip_malloc": (i32, [C.POINTER(vp), sz]),
    "tlm_hip_free": (i32, [vp]),
    "tlm_hip_memcpy_h2d": (i32, [vp, vp, sz, vp]),
    "tlm_hip_memcpy_d2h": (i32, [vp, vp, sz, vp]),
    "tlm_hip_sync": (i32, [vp]),
    "tlm_hip_qact_bytes": (sz, [i32, i64]),
    "tlm_hip_quantize_act": (i32, [i32, vp, i64, vp, vp]),
    "tlm_hip_expf": (i32, [vp, vp, i64, vp]),
    "tlm_hip_stream_read": (i32, [vp, sz, vp, vp]),
    "tlm_hip_matvec_rows": (i32, [i32, vp, sz, vp, vp, i64, i64, i64, vp]),
    "tlm_hip_packed_bytes": (sz, [i32, i64, i64]),
    "tlm_hip_pack": (i32, [i32, vp, sz, i64, i64, vp, vp]),
    "tlm_hip_matvec_packed": (i32, [i32, vp, i64, i64, vp, vp, vp]),
    "tlm_hip_mv_job": (i32, [C.POINTER(Seg), i32, vp]),
    "tlm_hip_matmul_tokens": (i32, [i32, vp, i64, i64, vp, i64, vp, vp]),
    "tlm_hip_moe_prefill_workspace_bytes": (sz, [C.POINTER(MoeDesc), i64]),
    "tlm_hip_moe_prefill": (i32, [C.POINTER(MoeDesc), vp, i64, vp, vp, vp, vp]),
    "tlm_hip_moe_workspace_bytes": (sz, [C.POINTER(MoeDesc)]),
    "tlm_hip_moe_layer": (i32, [C.POINTER(MoeDesc), vp, vp, vp, vp, vp]),
    "tlm_hip_moe_layer_noalloc": (i32, [C.POINTER(MoeDesc), vp, vp, vp, vp]),
    "tlm_hip_moe_layer_phase": (i32, [C.POINTER(MoeDesc), i32, vp, vp, vp, vp, vp]),
    "tlm_kern_hip_fill": (i32, [C.POINTER(QuantKernels)]),
    "tlm_hip_store_open": (i32, [C.POINTER(ExpertSrc), i32, C.POINTER(StoreOpts), C.POINTER(vp)]),
    "tlm_hip_store_close": (None, [vp]),
    "tlm_hip_store_n_slots": (i32, [vp]),
    "tlm_hip_store_slot_bytes": (C.c_uint64, [vp]),
    "tlm_hip_store_warm": (i32, [vp]),
    "tlm_hip_store_acquire": (i32, [vp, i32, C.POINTER(C.c_int), i32, C.POINTER(ExpertRef)]),
    "tlm_hip_store_wait": (i32, [vp, C.POINTER(ExpertRef)]),
    "tlm_hip_store_stream_wait": (i32, [vp, C.POINTER(ExpertRef), vp]),
    "tlm_hip_store_is_ready": (i32, [vp, C.POINTER(ExpertRef)]),
    "tlm_hip_store_release": (None, [vp, C.POINTER(ExpertRef), vp]),
    "tlm_hip_store_prefetch": (None, [vp, i32, C.POINTER(C.c_int), i32]),
    "tlm_hip_store_tick": (None, [vp]),
    "tlm_hip_store_drain": (i32, [vp]),
    "tlm_hip_store_get_stats": (None, [vp, C.POINTER(StoreStats)]),
    "tlm_hip_moe_route": (i32, [C.POINTER(MoeDesc), vp, vp, vp, vp, vp]),
    "tlm_hip_manifest_load": (i32, [C.c_char_p, C.POINTER(vp)]),
    "tlm_hip_manifest_free": (None, [vp]),
    "tlm_hip_manifest_geom": (C.POINTER(ModelGeom), [vp]),
    "tlm_hip_manifest_name": (C.c_char_p, [vp]),
    "tlm_hip_manifest_n_packets": (i32, [vp]),
    "tlm_hip_manifest_packet": (C.POINTER(PacketLoc), [vp, i32]),
    "tlm_hip_manifest_find": (C.POINTER(PacketLoc), [vp, i32, i32, C.c_uint32]),
    "tlm_hip_manifest_drive_path": (C.c_char_p, [vp, i32]),
    "tlm_hip_packet_read": (i32, [vp, C.POINTER(PacketLoc), vp, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "tlm_hip_packet_header": (i32, [vp, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]),
    "tlm_hip_dir_find": (i32, [vp, C.c_uint64, C.c_char_p, C.POINTER(TensorRef)]),
    "tlm_hip_model_open": (i32, [C.c_char_p, vp, C.POINTER(vp)]),
    "tlm_hip_model_synth": (i32, [C.POINTER(ModelGeom), C.POINTER(ModelSynthOpts), vp, C.POINTER(vp)]),
    "tlm_hip_model_close": (None, [vp]),
    "tlm_hip_model_geom_of": (C.POINTER(ModelGeom), [vp]),
    "tlm_hip_model_kv_len": (i32, [vp]),
    "tlm_hip_model_kv_capacity": (i32, [vp]),
    "tlm_hip_model_routes": (i32, [vp, vp, vp]),
    "tlm_hip_model_rewind": (i32, [vp, i32]),
    "tlm_hip_model_decode": (i32, [vp, i32]),
    "tlm_hip_model_sync": (i32, [vp]),
    "tlm_hip_model_stream": (vp, [vp]),
    "tlm_hip_model_expert_store": (vp, [vp]),
    "tlm_hip_model_get_stats": (i32, [vp, vp]),
    "tlm_hip_model_reset_stats": (None, [vp]),
    "tlm_hip_model_reset": (None, [vp]),
    "tlm_hip_model_step": (i32, [vp, i32, vp, C.POINTER(C.c_int32)]),
    "tlm_hip_model_generate": (i32, [vp, C.POINTER(C.c_int32), i32, i32, C.POINTER(C.c_int32)]),
    "tlm_hip_model_prefill": (i32, [vp, C.POINTER(C.c_int32), i32, vp]),
    "tlm_hip_model_prefill_batched": (i32, [vp]),
    "tlm_hip_crc32c": (C.c_uint32, [C.c_uint32, vp, sz]),
    "tlm_hip_sha256": (None, [vp, sz, vp]),
    "tlm_hip_moe_layer_store": (i32, [C.POINTER(MoeDesc), vp, i32, vp, vp, vp, C.POINTER(MoeHint), i32, vp, vp]),
    "tlm_hip_moe_stack_workspace_bytes": (sz, [C.POINTER(MoeDesc), i32, C.POINTER(StackOpts)]),
    "tlm_hip_moe_stack_store": (i32, [C.POINTER(MoeDesc), i32, vp, vp, C.POINTER(StackOpts), vp, vp, vp, vp]),
}

for _name, (_res, _args) in _SIGS.items():
    _f = getattr(lib, _name)
    _f.restype = _res
    _f.argtypes = _args

EXPORTS = tuple(_SIGS)


# return codes (include/tlm_hip.h; the reference's TLM_E* values)
TLM_HIP_OK, TLM_HIP_EIO, TLM_HIP_ENOMEM, TLM_HIP_EINVAL = 0, -1, -2, -3
TLM_HIP_EFORMAT, TLM_HIP_ERANGE, TLM_HIP_ENOTFOUND, TLM_HIP_EUNSUP, TLM_HIP_EBUSY = -4, -5, -6, -7, -8


class HipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"tlm_hip error {code}: {msg}")
        self.code = code


def check(rc):
    if rc != 0:
        raise HipError(rc, (lib.tlm_hip_errmsg() or b"").decode(errors="replace"))
    return rc
