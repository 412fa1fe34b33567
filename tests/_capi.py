"""ctypes bindings of the C ABI (include/graspo_tokpath.h), as a caller
without torch's extension would write them: plain pointers and sizes, device
buffers owned by the caller, the stream passed as a handle.  Tests use torch
only to allocate device memory and to read the results back."""

from __future__ import annotations

import ctypes

import torch

import graspo_amd

VP, I64, I32, SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t


class SamplerParams(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_int32),
                ("top_p", ctypes.c_float), ("repetition_penalty", ctypes.c_float)]


_SAMPLE_ARGS = [VP, I32, I64, I64, I64, VP, I64, I64, VP, I64, VP,
                ctypes.POINTER(SamplerParams), VP, I64, VP, VP, VP, VP, VP, VP, VP]


def lib() -> ctypes.CDLL:
    L = ctypes.CDLL(graspo_amd.LIB_PATH)
    L.gtp_sample_rows.argtypes = _SAMPLE_ARGS + [VP, SZ, VP]
    L.gtp_sample_rows.restype = I32
    L.gtp_sample_rows_noalloc.argtypes = _SAMPLE_ARGS + [VP]
    L.gtp_sample_rows_noalloc.restype = I32
    L.gtp_sample_workspace_bytes.argtypes = [I32, I64, I64, ctypes.POINTER(SamplerParams)]
    L.gtp_sample_workspace_bytes.restype = SZ
    L.gtp_logprob_entropy_rows.argtypes = [VP, I32, I64, I64, I64, VP, I32, VP, VP, VP, VP]
    L.gtp_logprob_entropy_rows.restype = I32
    L.gtp_decode_update_rows.argtypes = [VP, VP, I64, I64, I64, VP, VP, I64, VP, I64, I64, VP,
                                         VP]
    L.gtp_decode_update_rows.restype = I32
    L.gtp_sample_route.argtypes = [I32, I64, I64, I32, I64, I32, ctypes.POINTER(SamplerParams),
                                   SZ, ctypes.POINTER(ctypes.c_int32),
                                   ctypes.POINTER(ctypes.c_int32)]
    L.gtp_sample_route.restype = I32
    return L


ROUTE_SPLIT_TOPK, ROUTE_TOPP_SPLIT, ROUTE_TOPP, ROUTE_TOPP32, ROUTE_HIST, ROUTE_ROWWISE = range(1, 7)
NOALLOC_SCRATCH_BYTES = 8 << 20


def route(L, dtype, B, V, *, T, k=0, P=1.0, rho=1.0, hist_len=0, mask=False, aligned=True,
          workspace=None):
    """(route, slices) from gtp_sample_route; workspace None: the bytes
    gtp_sample_workspace_bytes asks for (what the torch op passes)."""
    p = SamplerParams(T, k, P, rho)
    ws = L.gtp_sample_workspace_bytes(dtype, B, V, ctypes.byref(p)) if workspace is None else workspace
    r, s = ctypes.c_int32(0), ctypes.c_int32(0)
    rc = L.gtp_sample_route(dtype, B, V, int(aligned), hist_len, int(mask), ctypes.byref(p), ws,
                            ctypes.byref(r), ctypes.byref(s))
    assert rc == 0
    return r.value, s.value


DTYPE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def stream_handle() -> int:
    return torch.cuda.current_stream().cuda_stream


class SampleBuffers:
    """Caller-owned output buffers of one sampler call."""

    def __init__(self, B: int, dev):
        self.ids = torch.full((B,), -7, dtype=torch.int64, device=dev)
        self.logprob = torch.empty(B, dtype=torch.float32, device=dev)
        self.sampled_logprob = torch.empty(B, dtype=torch.float32, device=dev)
        self.kept = torch.empty(B, dtype=torch.int32, device=dev)
        self.thresh_value = torch.empty(B, dtype=torch.float32, device=dev)
        self.thresh_id = torch.empty(B, dtype=torch.int32, device=dev)
        self.status = torch.full((B,), -7, dtype=torch.int32, device=dev)

    def out_args(self):
        return [ptr(self.ids), ptr(self.logprob), ptr(self.sampled_logprob), ptr(self.kept),
                ptr(self.thresh_value), ptr(self.thresh_id), ptr(self.status)]

    def cpu(self):
        return {k: v.cpu() for k, v in vars(self).items()}


def sample_args(logits: torch.Tensor, *, temperature, top_k=0, top_p=1.0,
                repetition_penalty=1.0, history=None, allow_mask=None, uniforms=None,
                finished=None, pad_token_id=0):
    """Leading arguments of gtp_sample_rows / _noalloc for [B, V] logits with
    unit-stride rows (history and mask contiguous, finished uint8 or bool);
    returns (args, params, B)."""
    B, V = logits.shape
    p = SamplerParams(float(temperature), int(top_k), float(top_p), float(repetition_penalty))
    hist_len = 0 if history is None else history.shape[1]
    mask_stride = 0 if allow_mask is None else allow_mask.shape[1]
    args = [ptr(logits), DTYPE[logits.dtype], B, V, logits.stride(0), ptr(history), hist_len,
            hist_len, ptr(allow_mask), mask_stride, ptr(uniforms), ctypes.byref(p),
            ptr(finished), int(pad_token_id)]
    return args, p, B


def sample_small_workspace(logits: torch.Tensor, **kw):
    """gtp_sample_rows with a fresh zeroed workspace of 256 bytes, too small
    for the split top-p kernel: a top-p call then takes the one-workgroup
    top-p kernel whatever B is.  Returns the outputs on the CPU as a dict of
    the SampleOutput fields."""
    L = lib()
    dev = logits.device
    args, p, B = sample_args(logits, **kw)
    nbytes = 256
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    out = SampleBuffers(B, dev)
    rc = L.gtp_sample_rows(*args, *out.out_args(), ws.data_ptr(), nbytes, stream_handle())
    assert rc == 0, rc
    torch.cuda.synchronize()
    return out.cpu()
