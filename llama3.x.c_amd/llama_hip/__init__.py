"""Python view of libllama3x_hip.so, the llama3.x.c matmul hot path on an MI355X.

The C ABI is declared in include/llama_hip*.h; this module only loads the library, declares the entry points' argument
types and mirrors the reference's structs (K8Weight, K8Input, GemmSegment, GemmQ8Segment, GemmBf16Segment,
AlignedBuffer, Config, Model), so callers write the same calls a C caller writes. Arguments that are buffers accept a
numpy array (host memory: the call copies in and out and waits), a torch CUDA tensor (device memory: used in place,
stream-ordered), an integer address, or None.

The library must be built (make -C llama3.x.c_amd, or __graft_entry__.build()); loading fails loudly otherwise. There is
no CPU fallback: on a machine without an MI355X every compute entry point fails with a message.
"""
import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "libllama3x_hip.so")
INCLUDE = os.path.join(ROOT, "include")

P = ctypes.c_void_p
I32 = ctypes.c_int
SZ = ctypes.c_size_t

# include/llama_hip_kernels.h: KernelIsa, KernelEpilogue
KERNELS_SCALAR, KERNELS_AVX512, KERNELS_AMX, KERNELS_HIP = 0, 1, 2, 3
K_STORE, K_ADD, K_PARTIAL, K_SWIGLU = 0, 1, 2, 3
# include/llama_hip_gemm.h: GemmKind, Q8GemmBackend
GEMM_STORE, GEMM_ADD, GEMM_SWIGLU, GEMM_PARTIAL = 0, 1, 2, 3
Q8_GEMM_PORTABLE, Q8_GEMM_AVX512, Q8_GEMM_AMX, Q8_GEMM_HIP_MFMA = 0, 1, 2, 3
# include/llama_hip.h
LLHIP_FAIL_EXIT, LLHIP_FAIL_RECORD = 0, 1
LOGITS_NONE, LOGITS_LAST, LOGITS_ALL = 0, 1, 2


class K8Weight(ctypes.Structure):
    _fields_ = [("q", P), ("s", P)]


class K8Input(ctypes.Structure):
    _fields_ = [("q", P), ("s", P), ("f", P)]


class GemmSegment(ctypes.Structure):
    _fields_ = [("c", P), ("ldc", I32), ("w", P), ("w3", P), ("ldw", SZ), ("n", I32), ("kind", I32)]


class GemmBf16Segment(ctypes.Structure):
    _fields_ = [("c", P), ("ldc", I32), ("w", P), ("w3", P), ("n", I32), ("kind", I32)]


class GemmQ8Segment(ctypes.Structure):
    _fields_ = [("c", P), ("ldc", I32), ("w", K8Weight), ("w3", K8Weight), ("pw", P), ("pw3", P), ("n", I32),
                ("kind", I32)]


class AlignedBuffer(ctypes.Structure):
    _fields_ = [("base", P), ("data", P), ("bytes", SZ)]


class PackBf16(ctypes.Structure):
    _fields_ = [("dst", P), ("w", P), ("rows", I32), ("cols", I32), ("ld", SZ)]


class PackS8(ctypes.Structure):
    _fields_ = [("dst", P), ("w", P), ("rows", I32), ("cols", I32), ("ld", SZ)]


DT_F32, DT_Q8 = 0, 1
SHARD_ROWS, SHARD_COLS, SHARD_COPY, SHARD_GLOBAL = 0, 1, 2, 3


class TensorDesc(ctypes.Structure):
    _fields_ = [("role", I32), ("layer", I32), ("rows", I32), ("cols", I32), ("dtype", I32), ("group_size", I32),
                ("offset", SZ), ("scale_offset", SZ), ("bytes", SZ), ("alias_of", I32)]


class Shard(ctypes.Structure):
    _fields_ = [("src", ctypes.POINTER(TensorDesc)), ("kind", I32), ("socket", I32), ("row0", I32), ("rows", I32),
                ("col0", I32), ("cols", I32), ("alias", I32), ("q_offset", SZ), ("s_offset", SZ), ("q", P),
                ("s", P), ("ld", SZ)]


class Config(ctypes.Structure):
    _fields_ = [(f, I32) for f in ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size", "seq_len",
                                   "format", "max_seq_len", "shared", "head_dim")] + \
               [(f, ctypes.c_float) for f in ("norm_eps", "rope_theta", "rope_factor", "rope_low", "rope_high")] + \
               [(f, I32) for f in ("rope_type", "rope_original", "bos_id", "eos_id", "eot_id", "eom_id")] + \
               [("name", ctypes.c_char * 128)]


class KvStats(ctypes.Structure):  # include/llama_hip_engine.h (runtime.h:80-86)
    _fields_ = [("reserved_bytes", SZ), ("active_bytes", SZ), ("resident_bytes", SZ), ("node", I32),
                ("verified", I32), ("full", I32), ("pages_queried", SZ), ("pages_wrong_node", SZ),
                ("pages_missing", SZ)]


class Model(ctypes.Structure):
    _fields_ = [("config", Config), ("implementation", P), ("file_bytes", SZ), ("mapped_bytes", SZ),
                ("max_batch", I32), ("prefill_logits", I32), ("prefill_gemm", I32), ("prefill_kernel", ctypes.c_char_p),
                ("prefill_bf16", I32)]


RowsDoneFn = ctypes.CFUNCTYPE(None, P, I32, I32)
SegmentFn = ctypes.CFUNCTYPE(None, P, I32, I32, I32)
FailFn = ctypes.CFUNCTYPE(None, ctypes.c_char_p)

class AttentionWork(ctypes.Structure):  # kernels.h:127-132
    _fields_ = [("partial", P), ("max_chunks", I32), ("n_heads", I32), ("head_dim", I32), ("workers", I32),
                ("external", I32), ("capacity", SZ)]


_SIGNATURES = {
    # the forward around the matmuls (llama_hip_forward.h)
    "k_rmsnorm": (None, [P, P, P, I32, ctypes.c_float]),
    "k_rmsnorm_rows": (None, [P, P, P, I32, I32, ctypes.c_float]),
    "llhip_rmsnorm_quantize_rows": (None, [P, P, P, P, I32, I32, ctypes.c_float, I32]),
    "llhip_rope_kv_store_rows": (None, [P, SZ, P, P, SZ, P, SZ, I32, I32, I32, I32, P, P, I32, I32]),
    "llhip_attention_batch_quantize": (None, [P, P, I32, P, P, P, P, I32, I32, I32, I32, I32, I32]),
    "llhip_gemm_q8_swiglu_quantize": (I32, [P, P, I32, I32, I32, P, P, I32, P, P]),
    "k_rope_table": (None, [P, I32, P]),
    "k_rope_apply": (None, [P, P, P, I32, I32, I32]),
    "k_rope_apply_rows": (None, [P, SZ, P, SZ, P, SZ, I32, I32, I32, I32]),
    "kernels_kv_layout_head": (I32, []),
    "kernels_kv_layout_name": (ctypes.c_char_p, []),
    "kernels_kv_layout_select": (I32, [ctypes.c_char_p]),
    "k_kv_strides": (None, [I32, I32, I32, P, P]),
    "k_kv_store": (None, [P, P, SZ, I32, I32, I32, I32, I32]),
    "k_embed_q8_rows": (None, [P, P, P, P, I32, I32, I32, I32]),
    "k_embed_f32_rows": (None, [P, P, P, I32, I32, I32]),
    "placement_hbm_budget": (SZ, []),
    "engine_load": (None, [P, ctypes.c_char_p]),
    "engine_load_context": (None, [P, ctypes.c_char_p, I32]),
    "engine_forward": (ctypes.POINTER(ctypes.c_float), [P, I32, I32]),
    "engine_free": (None, [P]),
    "engine_forward_batch": (ctypes.POINTER(ctypes.c_float), [P, P, I32, I32, I32]),
    "engine_group_size": (I32, []),
    "engine_precision": (ctypes.c_char_p, []),
    "engine_kv_stats": (None, [P, I32, I32, P]),
    "llhip_hbm_claimed": (SZ, []),
    "k_attention_init": (None, [P, I32, I32, I32, I32]),
    "k_attention_bytes": (SZ, [I32, I32, I32, I32]),
    "k_attention_init_in": (None, [P, I32, I32, I32, I32, P]),
    "k_attention_bytes_rows": (SZ, [I32, I32, I32, I32, I32]),
    "k_attention_init_rows": (None, [P, I32, I32, I32, I32, I32, P]),
    "k_attention_chunk_count": (I32, [P, I32, I32]),
    "k_attention_free": (None, [P]),
    "k_attention": (None, [P, P, P, P, P, P, I32, I32, I32, I32, I32]),
    "k_attention_layout": (None, [P, P, P, P, P, P, I32, I32, I32, I32, I32, SZ, SZ]),
    "k_attention_batch": (None, [P, P, P, P, P, P, I32, I32, I32, I32, I32, I32]),
    "k_attention_batch_layout": (None, [P, P, P, P, P, P, I32, I32, I32, I32, I32, I32, SZ, SZ]),
    "k_attention_batch_layout_noalloc": (None, [P, P, P, P, P, P, I32, I32, I32, I32, I32, I32, SZ, SZ]),
    "k_attention_kv": (None, [P, P, P, P, P, P, I32, I32, I32, I32, I32]),
    "k_attention_batch_kv": (None, [P, P, P, P, P, P, I32, I32, I32, I32, I32, I32]),
    "kernels_attention_name": (ctypes.c_char_p, []),
    "kernels_attention_decode_name": (ctypes.c_char_p, []),
    "kernels_attention_select": (I32, [ctypes.c_char_p, ctypes.c_char_p]),
    # kernels.h surface
    "kernels_init": (None, []),
    "kernels_select": (I32, [I32]),
    "kernels_name": (ctypes.c_char_p, []),
    "kernels_set_team": (None, [P]),
    "kernels_set_thread_team": (None, [P]),
    "kernels_backend_init": (None, []),
    "kernels_backend_free": (None, []),
    "kernels_backend_name": (ctypes.c_char_p, []),
    "kernels_avx512_active": (I32, []),
    "kernels_amx_active": (I32, []),
    "kernels_select_amx_auto": (I32, []),
    "kernels_parallel_segments": (None, [I32, P, SegmentFn, P]),
    "k_matmul": (None, [P, P, P, I32, I32]),
    "k_matmul_add": (None, [P, P, P, I32, I32]),
    "k_matmul_qkv": (None, [P, P, P, P, P, P, P, I32, I32, I32]),
    "k_matmul_swiglu": (None, [P, P, P, P, I32, I32]),
    "k_matmul_ld": (None, [P, P, P, SZ, I32, I32, I32]),
    "k_matmul_ld_worker": (None, [P, P, P, SZ, I32, I32, I32, I32, I32, P, RowsDoneFn, P]),
    "k_matmul_swiglu_ld": (None, [P, P, P, P, SZ, I32, I32]),
    "k_quantize": (None, [P, P, P, I32, I32]),
    "k_matmul_q8": (None, [P, ctypes.POINTER(K8Input), K8Weight, I32, I32, I32]),
    "k_matmul_q8_add": (None, [P, ctypes.POINTER(K8Input), K8Weight, I32, I32, I32]),
    "k_matmul_q8_qkv": (None, [P, P, P, ctypes.POINTER(K8Input), K8Weight, K8Weight, K8Weight, I32, I32, I32, I32]),
    "k_matmul_q8_swiglu": (None, [P, ctypes.POINTER(K8Input), K8Weight, K8Weight, I32, I32, I32]),
    "k_matmul_q8_ld": (None, [P, ctypes.POINTER(K8Input), ctypes.POINTER(K8Weight), SZ, I32, I32, I32, I32]),
    "k_matmul_q8_ld_worker": (None, [P, ctypes.POINTER(K8Input), ctypes.POINTER(K8Weight), SZ, I32, I32, I32, I32, I32,
                                     I32, P, RowsDoneFn, P]),
    "k_matmul_q8_swiglu_ld": (None, [P, ctypes.POINTER(K8Input), ctypes.POINTER(K8Weight), ctypes.POINTER(K8Weight), SZ,
                                     I32, I32, I32]),
    "k_gemv_force_hybrid": (None, [I32]),
    # gemm.h surface
    "k_gemm_f32": (None, [P, I32, I32, I32, ctypes.POINTER(GemmSegment), I32]),
    "k_gemm_f32_portable": (None, [P, I32, I32, I32, ctypes.POINTER(GemmSegment), I32, I32]),
    "k_gemm_f32_simd_test": (I32, [P, I32, I32, I32, ctypes.POINTER(GemmSegment), I32, I32]),
    "k_gemm_kc": (I32, []),
    "gemm_amx_unavailable": (ctypes.c_char_p, []),
    "gemm_amx_permission": (ctypes.c_char_p, []),
    "gemm_amx_enable": (None, [I32]),
    "gemm_amx_active": (I32, []),
    "gemm_amx_emulated": (I32, []),
    "gemm_amx_thread_release": (None, []),
    "bf16_from_f32": (ctypes.c_uint16, [ctypes.c_float]),
    "f32_from_bf16": (ctypes.c_float, [ctypes.c_uint16]),
    "bf16_vnni_elements": (SZ, [I32, I32]),
    "s8_vnni_bytes": (SZ, [I32, I32]),
    "pack_bf16_vnni": (None, [P, P, I32, I32, SZ]),
    "pack_bf16_vnni_tiles": (None, [P, P, I32, I32, SZ, I32, I32]),
    "pack_s8_vnni": (None, [P, P, I32, I32, SZ]),
    "pack_s8_vnni_tiles": (None, [P, P, I32, I32, SZ, I32, I32]),
    "pack_bf16_vnni_many": (None, [P, I32]),
    "pack_s8_vnni_many": (None, [P, I32]),
    "pack_bf16_job_from_shard": (PackBf16, [P, ctypes.POINTER(Shard)]),
    "pack_s8_job_from_shard": (PackS8, [P, ctypes.POINTER(Shard)]),
    "amx_bf16_tile_gemm": (None, [P, SZ, P, SZ, P, I32, I32, I32]),
    "amx_s8_tile_gemm": (None, [P, SZ, P, SZ, P, I32, I32, I32]),
    "aligned_buffer_alloc": (None, [ctypes.POINTER(AlignedBuffer), SZ, I32]),
    "aligned_buffer_free": (None, [ctypes.POINTER(AlignedBuffer)]),
    "k_gemm_bf16_panel_bytes": (SZ, [I32, I32]),
    "k_gemm_bf16": (None, [P, I32, I32, I32, ctypes.POINTER(GemmBf16Segment), I32, ctypes.POINTER(AlignedBuffer)]),
    "k_quantize_rows": (None, [P, P, P, SZ, I32, I32, I32]),
    "k_gemm_q8": (None, [P, P, I32, I32, I32, ctypes.POINTER(GemmQ8Segment), I32]),
    "k_gemm_q8_pick": (I32, [I32, ctypes.POINTER(GemmQ8Segment), I32]),
    "k_gemm_q8_backend_test": (I32, [I32, P, P, I32, I32, I32, ctypes.POINTER(GemmQ8Segment), I32]),
    "llhip_q8_group_dots": (None, [P, P, I32, I32, I32, P, I32]),
    "k_gemm_q8_amx_dots_test": (I32, [P, P, I32, I32, I32, P, I32]),
    # prefill.h surface
    "prefill_precision": (I32, [I32]),
    "prefill_configure": (None, [ctypes.POINTER(Model), I32]),
    "prefill_configure_engine": (None, [ctypes.POINTER(Model), I32, I32]),
    "prefill_validate": (None, [ctypes.POINTER(Model), P, I32, I32, I32]),
    "engine_max_batch": (I32, [ctypes.POINTER(Model)]),
    # llama_hip.h device runtime
    "llhip_init": (I32, []),
    "llhip_device_name": (ctypes.c_char_p, []),
    "llhip_device_cu_count": (I32, []),
    "llhip_stream": (P, []),
    "llhip_synchronize": (None, []),
    "llhip_register_host": (I32, [P, SZ]),
    "llhip_unregister_host": (I32, [P]),
    "llhip_resolve": (P, [P]),
    "llhip_malloc": (P, [SZ]),
    "llhip_free": (None, [P]),
    "llhip_memcpy_h2d": (None, [P, P, SZ]),
    "llhip_memcpy_d2h": (None, [P, P, SZ]),
    "llhip_memcpy_d2d": (None, [P, P, SZ]),
    "llhip_graph_begin": (I32, []),
    "llhip_graph_end": (P, []),
    "llhip_graph_launch": (I32, [P]),
    "llhip_graph_destroy": (None, [P]),
    "llhip_set_fail_handler": (None, [P]),
    "llhip_set_fail_mode": (None, [I32]),
    "llhip_last_error": (ctypes.c_char_p, []),
    "llhip_clear_error": (None, []),
    "llhip_q8_gemv_group_dots": (None, [P, P, P, P, P, SZ, I32, I32, I32]),
    "llhip_set_gemv_shape": (None, [I32, I32, I32]),
    "llhip_set_gemm_splits": (None, [I32]),
    "llhip_set_bf16_tile": (None, [I32]),
    "llhip_set_q8_tile": (None, [I32]),
    "llhip_set_q8_scales": (None, [I32]),
}

_lib = None


def declared_functions():
    """Every function name include/llama_hip*.h declares (the exported C ABI)."""
    names = set()
    for fn in sorted(os.listdir(INCLUDE)):
        if fn.startswith("llama_hip") and fn.endswith(".h"):
            text = open(os.path.join(INCLUDE, fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(\w+)\s*\(([^;{]*)\)\s*;", text, flags=re.M):
                if not m.group(0).lstrip().startswith("typedef"):
                    names.add(m.group(1))
    return names


def load(path=None):
    """The library with every entry point's argument types declared. Raises if it is not built. LLAMA_HIP_LIB names
    another build of it (a variant under test) instead of the in-tree one."""
    global _lib
    if _lib is not None:
        return _lib
    path = path or os.environ.get("LLAMA_HIP_LIB") or LIB_PATH
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built: run make -C llama3.x.c_amd (or __graft_entry__.build())")
    # One HIP runtime per process: torch's libtorch_hip links its bundled libamdhip64.so by file name, while this
    # library asks for the soname libamdhip64.so.7, which an already-loaded copy satisfies. Loading torch first (when
    # it is installed) makes both use torch's copy; the other order would load two runtimes that do not share devices.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def ptr(x):
    """The address of a buffer argument: numpy array, torch tensor, integer, ctypes object, or None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if hasattr(x, "ctypes"):
        return x.ctypes.data
    return ctypes.cast(ctypes.pointer(x), P).value


def record_failures():
    """Switch to LLHIP_FAIL_RECORD: a failing call returns and keeps its message (llhip_last_error)."""
    lib = load()
    lib.llhip_set_fail_mode(LLHIP_FAIL_RECORD)
    lib.llhip_clear_error()


def last_error():
    msg = load().llhip_last_error()
    return msg.decode() if msg else ""


def k8(q, s, f=None):
    return K8Input(ptr(q), ptr(s), ptr(f))


def w8(q, s):
    return K8Weight(ptr(q), ptr(s))
