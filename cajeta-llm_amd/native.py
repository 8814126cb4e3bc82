"""ctypes binding of libcajeta_mi355x.so (include/cajeta_mi355x.h).

The same calls a Cajeta @Native binding makes: int32/int64/float scalars,
int64 handles and primitive arrays. Every non-OK status raises LlmException
with the library's message — a refused launch is never silent, and there is
no CPU fallback: without the built library or a GPU the calls fail loudly.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcajeta_mi355x.so")
HSACO_PATH = os.path.join(HERE, "kernels.hsaco")

P, I32, I64, F32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
CP = ctypes.c_char_p

# status codes (include/cajeta_mi355x.h)
CJ_OK, CJ_ERR_ARG, CJ_ERR_HIP, CJ_ERR_NOKERNEL, CJ_ERR_STATE, CJ_ERR_CAPACITY, CJ_ERR_IO = 0, -1, -2, -3, -4, -5, -6

# name: (restype, argtypes) — one entry per declaration in include/cajeta_mi355x.h
SIGNATURES = {
    "cj_init": (I32, [I32]),
    "cj_shutdown": (I32, []),
    "cj_last_error": (I32, [P, I32]),
    "cj_kernel_available": (I32, [CP]),
    "cj_device_info": (I32, [P, I32]),
    "cj_buf_alloc": (I64, [I64]),
    "cj_buf_free": (I32, [I64]),
    "cj_buf_size": (I64, [I64]),
    "cj_buf_upload": (I32, [I64, I64, P, I64]),
    "cj_buf_download": (I32, [I64, I64, P, I64]),
    "cj_buf_zero": (I32, [I64]),
    "cj_stream_sync": (I32, []),
    "cj_graph_begin": (I32, []),
    "cj_graph_end": (I64, []),
    "cj_graph_launch": (I32, [I64]),
    "cj_graph_free": (I32, [I64]),
    "cj_event_record": (I64, []),
    "cj_event_wait": (I32, [I64]),
    "cj_event_free": (I32, [I64]),
    "cj_q8k_pack": (I32, [I64, I64, I64, I64, I64, I32]),
    "cj_rmsnorm_pack": (I32, [I64, I64, I64, I64, I64, F32, I32, I32]),
    "cj_prepared_row_bytes": (I64, [I32, I64]),
    "cj_prepare_weight": (I32, [I64, I64, I32, I64, I64]),
    "cj_matvec": (I32, [I32, I64, I64, I64, I64, I64, I64, I32]),
    "cj_matvec_mxfp4_q8": (I32, [I64, I64, I64, I64, I64, I64, I32]),
    "cj_matmul": (I32, [I32, I64, I64, I64, I64, I64, I32, I64, I64, I64, I32]),
    "cj_glu": (I32, [I64, I64, I64, I64, I64, I32, I32]),
    "cj_add": (I32, [I64, I64, I64]),
    "cj_buf_copy": (I32, [I64, I64, I64]),
    "cj_rope_table": (I32, [I64, I32, F32, I32]),
    "cj_rope_table_freqs": (I32, [I64, I32, F32, I32, P, I32]),
    "cj_qk_prep": (I32, [I64, I64, I64, I64, I64, I64, I64, I64, I64, I32, I32, I32, I32, I32, F32, I32, I32]),
    "cj_attend": (I32, [I64, I64, I64, I64, I64, I64, I32, I64, I32, I32, I32, I32, I32, I32, F32]),
    "cj_decode_splits": (I32, [I32, I32, I32]),
    "cj_attn_merge": (I32, [I64, I64, I64, I32, I32, I32, I32]),
    "cj_embed_row": (I32, [I64, I64, I32, I64, I32]),
    "cj_argmax_row": (I32, [I64, I32, I64, I64]),
    "cj_dequant": (I32, [I64, I64, I32, I64, I64, I32]),
    "cj_moe_route": (I32, [I64, I64, I64, I32, I32, I32, I32, F32, I64]),
    "cj_embed_row_slot": (I32, [I64, I64, I32, I64, I32, I64, I32, I64]),
    "cj_argmax_row_noalloc": (I32, [I64, I32, I64, I64]),
    "cj_router_topk": (I32, [I64, I64, I64, I64, I64, I64, I32, I32, I32, I32, F32]),
    "cj_attn_scores": (I32, [I64, I64, I64, I64, I32, I32, I32, I32, I32, I32, F32]),
    "cj_engine_load": (I64, [CP, I32, I32]),
    "cj_engine_load_kv": (I64, [CP, I32, I32, I32, I32]),
    "cj_engine_close": (I32, [I64]),
    "cj_engine_config": (I32, [I64, P, I32]),
    "cj_engine_submit": (I32, [I64, P, I32, I32]),
    "cj_engine_submit_stops": (I32, [I64, P, I32, I32, P, I32]),
    "cj_engine_run_all": (I32, [I64, I32]),
    "cj_engine_step_once": (I32, [I64]),
    "cj_engine_request": (I32, [I64, I32, P, I32, P, P]),
    "cj_engine_cancel": (I32, [I64, I32]),
    "cj_engine_set_eog": (I32, [I64, P, I32]),
    "cj_engine_reset": (I32, [I64, I32]),
    "cj_engine_prefill": (I32, [I64, I32, P, I32]),
    "cj_engine_decode": (I32, [I64, I32, I32, P]),
    "cj_engine_decode_batch": (I32, [I64, P, I32, I32, P]),
    "cj_engine_set_prefill_chunk": (I32, [I64, I32]),
    "cj_engine_set_cpu_threads": (I32, [I64, I32]),
    "cj_engine_logits": (I32, [I64, I32, P, I64]),
    "cj_engine_preds": (I32, [I64, I32, P, I32]),
    "cj_engine_last_step_us": (F32, [I64]),
    "cj_engine_trace": (I32, [I64, I32, P, I64]),
    "cj_engine_time_kernel": (I32, [I64, I32, I32, I32, P, P, P, I32]),
    "cj_engine_time_kernel_in_step": (I32, [I64, I32, I32, I32, P]),
    "cj_engine_step_bytes": (I64, [I64, I32]),
    "cj_engine_set_graphs": (I32, [I64, I32]),
    "cj_synth_gguf": (I32, [CP, CP, I64]),
    "cj_image_info": (I32, [CP, P, P]),
    "cj_gguf_info": (I32, [CP, P, P]),
    "cj_image_free": (I32, [CP]),
}

TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K, TYPE_MXFP4 = 0, 1, 2, 8, 12, 14, 39


class LlmException(Exception):
    """The reference's LlmException (L/LlmException.cajeta): a named failure."""


_lib = None
_device = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH) or not os.path.exists(HSACO_PATH):
            raise LlmException("the MI355X backend is not built: run __graft_entry__.build() "
                               "(missing %s)" % (LIB_PATH if not os.path.exists(LIB_PATH) else HSACO_PATH))
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def last_error():
    buf = ctypes.create_string_buffer(1024)
    lib().cj_last_error(buf, 1024)
    return buf.value.decode(errors="replace")


def check(rc, what=""):
    """Raise on a negative status (or a zero handle when `what` says handle)."""
    if isinstance(rc, int) and rc < 0:
        raise LlmException("%s failed (%d): %s" % (what or "call", rc, last_error()))
    return rc


def handle(h, what):
    if not h:
        raise LlmException("%s failed: %s" % (what, last_error()))
    return h


def init(device=0):
    global _device
    if _device is None:
        check(lib().cj_init(device), "cj_init")
        _device = device
    return _device


def ptr(a):
    """numpy array -> void*"""
    return a.ctypes.data_as(ctypes.c_void_p)


class Buffer:
    """A device buffer (the reference's KernelBuffer<T>) by handle."""

    def __init__(self, nbytes):
        init()
        self.nbytes = int(nbytes)
        self.h = handle(lib().cj_buf_alloc(self.nbytes), "cj_buf_alloc(%d)" % self.nbytes)

    @classmethod
    def of(cls, array):
        import numpy as np
        a = np.ascontiguousarray(array)
        b = cls(max(a.nbytes, 16))
        b.upload(a)
        return b

    def upload(self, array, off=0):
        import numpy as np
        a = np.ascontiguousarray(array)
        check(lib().cj_buf_upload(self.h, off, ptr(a), a.nbytes), "cj_buf_upload")

    def download(self, dtype, count, off=0):
        import numpy as np
        out = np.empty(count, dtype)
        check(lib().cj_buf_download(self.h, off, ptr(out), out.nbytes), "cj_buf_download")
        return out

    def zero(self):
        check(lib().cj_buf_zero(self.h), "cj_buf_zero")

    def free(self):
        if self.h:
            lib().cj_buf_free(self.h)
            self.h = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sync():
    check(lib().cj_stream_sync(), "cj_stream_sync")
