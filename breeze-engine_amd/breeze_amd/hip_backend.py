"""ctypes bridge to the gfx950 quantized linear library.

Drop-in for ``breeze.cpu_backend`` (breeze/cpu_backend.py:57-242): the same
``available / set_threads / set_hi_prec / prepack / matmul / free`` surface,
argument order, validation and exceptions, over ``libbreeze_qmm.so``, whose
C ABI keeps the reference's ``i4_*`` names (include/breeze_qmm.h).

GPU additions: ``matmul`` also takes a PyTorch-ROCm tensor on the GPU and
returns one (computed on the current stream, no host round trip);
``matmul_argmax`` adds the LM-head argmax; ``unpack`` and ``block_dots``
expose the packed handle and the exact block integers for tests.

There is no CPU fallback: without the library or a gfx950 device the calls
raise.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.environ.get("BREEZE_HIP_KERNEL", os.path.join(_HERE, "libbreeze_qmm.so"))

_vp = ctypes.c_void_p
_i = ctypes.c_int

_lib = None
_native_prepack = None


def _bind_torch_runtime():
    """Load PyTorch's own HIP runtime (by path, without importing torch) before
    the library, so the library's libamdhip64.so.7 dependency resolves to it.

    PyTorch-ROCm ships its own libamdhip64/libhsa-runtime64 and asks for them
    by a name that does not match the system runtime's soname; if the system
    runtime were loaded first the process would hold two HSA runtimes and
    only the first to initialise would see the GPU."""
    import importlib.util

    try:
        spec = importlib.util.find_spec("torch")
    except (ImportError, ValueError):
        return
    for d in (spec.submodule_search_locations or []) if spec else []:
        path = os.path.join(d, "lib", "libamdhip64.so")
        if os.path.exists(path):
            ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
            return


if os.environ.get("BREEZE_HIP_SYSTEM_RUNTIME") != "1":
    try:
        _bind_torch_runtime()
    except OSError:
        pass

try:
    _lib = ctypes.CDLL(_SO)
    _lib.i4_prepack.restype = _vp
    _lib.i4_prepack.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _i]
    _lib.i4_matmul.argtypes = [_vp, _vp, _i, _vp]
    _lib.i4_matmul.restype = None
    _lib.i4_matmul_region.argtypes = [_vp, _vp, _i, _vp, _vp, _vp]
    _lib.i4_matmul_region.restype = None
    _lib.i4_free.argtypes = [_vp]
    _lib.i4_free.restype = None
    for _name in ("i4_set_threads", "i4_set_hi_prec", "i4_set_numa_split"):
        getattr(_lib, _name).argtypes = [_i]
        getattr(_lib, _name).restype = None
    _lib.i4_last_error.restype = ctypes.c_char_p
    _lib.i4_last_error.argtypes = []
    _lib.i4_device_ok.restype = _i
    _lib.i4_device_ok.argtypes = []
    _lib.i4_matmul_dev.restype = _i
    _lib.i4_matmul_dev.argtypes = [_vp, _vp, _i, _vp, _vp]
    _lib.i4_matmul_argmax_dev.restype = _i
    _lib.i4_matmul_argmax_dev.argtypes = [_vp, _vp, _i, _vp, _vp, _vp]
    _lib.i4_matmul_noalloc_dev.restype = _i
    _lib.i4_matmul_noalloc_dev.argtypes = [_vp, _vp, _i, _vp, _vp, _vp]
    _lib.i4_matmul_multi_dev.restype = _i
    _lib.i4_matmul_multi_dev.argtypes = [_vp, _i, _vp, _i, _vp, _vp]
    _lib.i4_rmsnorm_matmul_multi_dev.restype = _i
    _lib.i4_rmsnorm_matmul_multi_dev.argtypes = [_vp, _vp, ctypes.c_float, _vp, _i, _i, _vp, _vp, _vp]
    _lib.i4_matmul_silu_mul_dev.restype = _i
    _lib.i4_matmul_silu_mul_dev.argtypes = [_vp, _vp, _vp, _i, _vp, _vp]
    _lib.i4_silu_mul_dev.restype = _i
    _lib.i4_silu_mul_dev.argtypes = [_vp, _vp, ctypes.c_size_t, _vp, _vp]
    _lib.i4_block_dots_dev.restype = _i
    _lib.i4_block_dots_dev.argtypes = [_vp, _vp, _i, _vp, _vp]
    _lib.i4_plan_query.restype = _i
    _lib.i4_plan_query.argtypes = [_i, _i, _i, _i, _i, _i, _vp, _i]
    _lib.i4_handle_info.restype = _i
    _lib.i4_handle_info.argtypes = [_vp, _vp]
    _lib.i4_unpack.restype = _i
    _lib.i4_unpack.argtypes = [_vp, _vp, _vp, _vp, _vp]
    _lib.i4_rmsnorm_dev.restype = _i
    _lib.i4_rmsnorm_dev.argtypes = [_vp, _vp, _i, _i, ctypes.c_float, _vp, _vp]
except (OSError, AttributeError):
    _lib = None

if _lib is not None:
    _native_prepack = _lib.i4_prepack_onnx
    _native_prepack.restype = _vp
    _native_prepack.argtypes = [_vp] * 3 + [_i] * 4


def available():
    """True when the library is loaded (compute additionally needs a GPU)."""
    return _lib is not None


def device_available():
    """True when the library is loaded and a gfx950 device can run it."""
    return _lib is not None and _lib.i4_device_ok() == 1


def last_error():
    return _lib.i4_last_error().decode() if _lib is not None else "library not loaded"


def set_threads(n):
    """Accepted for API compatibility; the GPU path has no host thread pool."""
    if _lib is not None:
        _lib.i4_set_threads(int(n))


def set_hi_prec(on):
    """Select process-global INT16 two-pass (on) or INT8 activation quantization.

    Configure before inference; like the reference, concurrent mutation is not
    thread-safe and callers serialize setting changes with native work."""
    if _lib is not None:
        _lib.i4_set_hi_prec(1 if on else 0)


def _p(a):
    return a.ctypes.data_as(_vp) if a is not None else None


def _require_lib():
    if _lib is None:
        raise RuntimeError(f"GPU kernel library unavailable ({_SO}); build it with "
                           "`python -m breeze_amd._build`")


def prepack(qweight, scales, qzeros, K, N, bits=4, block_size=32):
    """Pack ONNX MatMulNBits weights into device memory; returns an int handle.

    Same contract as breeze/cpu_backend.py:119-168: 4-bit (nibbles, zero
    point default 8) or 8-bit (bytes, symmetric zero point 128) weights in
    blocks of 32; scales fp16 are kept as fp16 bits, anything else is
    converted to fp32; the handle owns device copies of everything."""
    if bits not in (4, 8) or block_size != 32:
        raise ValueError("quantized prepack requires 4/8-bit weights and block_size=32")
    if (not isinstance(N, (int, np.integer)) or not isinstance(K, (int, np.integer))
            or isinstance(N, (bool, np.bool_)) or isinstance(K, (bool, np.bool_))
            or N > np.iinfo(np.int32).max or K > np.iinfo(np.int32).max):
        raise ValueError("Prepack dimensions must be signed 32-bit integers")
    N, K = int(N), int(K)
    if N <= 0 or K <= 0 or N % 16 or K % 32:
        raise ValueError(f"need N%16==0,K%32==0 (got N={N},K={K})")
    qweight = np.asarray(qweight)
    if qweight.dtype != np.uint8:
        raise ValueError("MatMulNBits packed weights must be uint8")
    nblk = K // 32
    if qweight.size != N * nblk * (4 * bits):
        raise ValueError("Incorrect packed weight size for the supplied dimensions")
    scales = np.asarray(scales)
    if scales.size != N * nblk:
        raise ValueError("Incorrect scale count for the supplied dimensions")
    if qzeros is not None and np.size(qzeros):
        qzeros = np.asarray(qzeros)
        if qzeros.dtype != np.uint8:
            raise ValueError("Packed zero points must be uint8")
        if qzeros.size != N * (nblk if bits == 8 else (nblk + 1) // 2):
            raise ValueError("Incorrect zero-point count for the supplied dimensions")
        if bits == 8 and np.any(qzeros != 128):
            raise ValueError("INT8 weights require symmetric zero point 128")
        qzeros = np.ascontiguousarray(qzeros) if bits == 4 else None
    else:
        qzeros = None
    _require_lib()
    if _native_prepack is None:
        return _prepack_numpy(qweight, scales, qzeros, K, N, bits, block_size)

    qw = np.ascontiguousarray(qweight)
    scale_dtype = np.float16 if scales.dtype == np.float16 else np.float32
    sc = np.require(scales, dtype=scale_dtype, requirements=["C", "A"])
    handle = _native_prepack(_p(qw), _p(sc), _p(qzeros), N, K, int(bits), sc.itemsize * 8)
    if not handle:
        raise MemoryError(f"Could not allocate packed {bits}-bit weights (N={N}, K={K}): "
                          f"{last_error()}")
    return handle


def _legacy_layout(qweight, scales, qzeros, K, N, bits=4):
    """MatMulNBits -> the reference's legacy pre-transformed layout, in NumPy
    (the layout breeze/cpu_backend.py:171-227 builds): tiles of 16 columns,
    per 32-block 8 groups of 4 k; INT8 signed bytes [N/16, nblk, 8, 64],
    INT4 nibble pairs [N/16, nblk, 8, 32]; scale, zp (INT4) and
    corr = 128 * (sum(q) - 32 * zp) as [N/16, nblk, 16].
    Returns (B, scale, zp or None, corr)."""
    nblk = K // 32
    ntiles = N // 16

    def tile16(x):  # [N, nblk] -> [ntiles, nblk, 16]
        return np.ascontiguousarray(x.reshape(ntiles, 16, nblk).transpose(0, 2, 1))

    sc = tile16(np.asarray(scales, dtype=np.float32).reshape(N, nblk))
    if bits == 8:
        w = np.ascontiguousarray(qweight).reshape(N, nblk, 32).astype(np.int16)
        b = (w - 128).astype(np.int8)
        Bv = np.ascontiguousarray(
            b.reshape(ntiles, 16, nblk, 8, 4).transpose(0, 2, 3, 1, 4).reshape(ntiles, nblk, 8, 64))
        corr = tile16((128 * b.astype(np.int32).sum(axis=2)).astype(np.int32))
        return Bv, sc, None, corr
    qw = np.ascontiguousarray(qweight).reshape(N, nblk, 16)
    w = np.empty((N, nblk, 32), np.uint8)
    w[:, :, 0::2] = qw & 15
    w[:, :, 1::2] = qw >> 4
    if qzeros is not None and np.size(qzeros):
        packed = (nblk + 1) // 2
        qz = np.ascontiguousarray(qzeros).reshape(N, packed)
        zpf = np.empty((N, packed * 2), np.uint8)
        zpf[:, 0::2] = qz & 15
        zpf[:, 1::2] = qz >> 4
        zp = zpf[:, :nblk].astype(np.int32)
    else:
        zp = np.full((N, nblk), 8, np.int32)
    w2 = w.reshape(ntiles, 16, nblk, 8, 4).transpose(0, 2, 3, 1, 4).reshape(ntiles, nblk, 8, 64)
    Bv = np.ascontiguousarray((w2[..., 0::2] | (w2[..., 1::2] << 4)).astype(np.uint8))
    zp_t = tile16(zp.astype(np.int8))
    corr = tile16((128 * (w.astype(np.int32).sum(axis=2) - 32 * zp)).astype(np.int32))
    return Bv, sc, zp_t, corr


def _prepack_numpy(qweight, scales, qzeros, K, N, bits=4, block_size=32):
    """Pack through the legacy entry point ``i4_prepack`` from the layout
    ``_legacy_layout`` builds.  Callers validate the contract first.  Tests
    use it to show the legacy and MatMulNBits entry points agree."""
    _require_lib()
    Bv, sc, zp, corr = _legacy_layout(qweight, scales, qzeros, K, N, bits)
    handle = _lib.i4_prepack(_p(Bv), _p(sc), _p(zp), _p(corr), N, K, K // 32, bits)
    if not handle:
        raise MemoryError(f"Could not allocate packed {bits}-bit weights (N={N}, K={K}): "
                          f"{last_error()}")
    return handle


def _is_torch(x):
    return type(x).__module__.split(".")[0] == "torch"


def _torch_stream(t):
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _check_rc(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed ({rc}): {last_error()}")


def matmul(handle, a2d, N):
    """a2d: fp32 [M, K].  Returns fp32 [M, N].

    NumPy in, NumPy out (blocking, like the reference); a GPU torch tensor in,
    a GPU torch tensor out (asynchronous on the current stream)."""
    _require_lib()
    if _is_torch(a2d):
        import torch
        a = a2d.to(torch.float32).contiguous()
        M = a.shape[0]
        out = torch.empty((M, N), dtype=torch.float32, device=a.device)
        _check_rc(_lib.i4_matmul_dev(_vp(handle), _vp(a.data_ptr()), int(M), _vp(out.data_ptr()),
                                     _torch_stream(a)), "i4_matmul_dev")
        return out
    a2d = np.ascontiguousarray(a2d, dtype=np.float32)
    M = a2d.shape[0]
    out = np.empty((M, N), dtype=np.float32)
    _lib.i4_matmul(_vp(handle), _p(a2d), int(M), _p(out))
    err = last_error()
    if err:
        raise RuntimeError(f"i4_matmul failed: {err}")
    return out


def matmul_silu_mul(gate, up, a2d, N):
    """GPU torch tensor [M, K] -> silu(a @ Wgate) * (a @ Wup), fp32 [M, N]: the
    decoder MLP's gate/up step (kernel/qwen35_decoder.cpp:406-408) in one
    call, asynchronous on the current stream."""
    _require_lib()
    import torch
    a = a2d.to(torch.float32).contiguous()
    M = a.shape[0]
    out = torch.empty((M, N), dtype=torch.float32, device=a.device)
    _check_rc(_lib.i4_matmul_silu_mul_dev(_vp(gate), _vp(up), _vp(a.data_ptr()), int(M), _vp(out.data_ptr()),
                                          _torch_stream(a)), "i4_matmul_silu_mul_dev")
    return out


PLAN_FIELDS = ("route", "quant", "fused", "p64", "lrec", "rows_per_group", "row_groups", "tile_ranges", "pair_xcd",
               "lds", "pf_rp", "pf_ct", "grid_x", "grid_y", "split", "stream", "flow")
ROUTES = {0: None, 1: "decode", 2: "decode8", 3: "prefill", 4: "rows"}
QUANTIZERS = {0: None, 1: "staged", 2: "rows8", 3: "prefill"}


def plan(bits, M, K, N, n_cu=256, dots=False, argmax=False, pair=False, multi=False, norm=False, extra=False,
         legacy_corr=False):
    """The library's routing decision for a call (i4_plan_query), without a
    device: which kernel, which stand-alone quantizer and the launch shape."""
    _require_lib()
    flags = (1 * dots) | (2 * argmax) | (4 * pair) | (8 * multi) | (16 * norm) | (32 * extra) | (64 * legacy_corr)
    out = np.zeros(len(PLAN_FIELDS), np.int32)
    n = _lib.i4_plan_query(int(bits), int(M), int(K), int(N), flags, int(n_cu), _p(out), len(out))
    if n < 0:
        raise ValueError(f"i4_plan_query: {last_error()}")
    d = dict(zip(PLAN_FIELDS, (int(v) for v in out)))
    d["route"] = ROUTES[d["route"]]
    d["quant"] = QUANTIZERS[d["quant"]]
    return d


def silu_mul(g, u):
    """GPU torch tensors g, u (same shape, fp32) -> silu(g) * u, the decoder
    MLP's elementwise step (kernel/qwen35_decoder.cpp:408) bit for bit,
    asynchronous on the current stream."""
    _require_lib()
    import torch
    g = g.to(torch.float32).contiguous()
    u = u.to(torch.float32).contiguous()
    if g.shape != u.shape:
        raise ValueError(f"silu_mul: shapes {tuple(g.shape)} and {tuple(u.shape)} differ")
    out = torch.empty_like(g)
    _check_rc(_lib.i4_silu_mul_dev(_vp(g.data_ptr()), _vp(u.data_ptr()), g.numel(), _vp(out.data_ptr()),
                                   _torch_stream(g)), "i4_silu_mul_dev")
    return out


def matmul_multi(handles, a2d, Ns):
    """GPU torch tensor [M, K] -> [a @ W_i for each handle] (fp32 [M, N_i]):
    projections of one activation, e.g. the decoder's in_qkv, in_z, in_b,
    in_a (kernel/qwen35_decoder.cpp:285-288), in one launch when they share
    a device layout; asynchronous on the current stream."""
    _require_lib()
    import torch
    if not 1 <= len(handles) <= 4 or len(handles) != len(Ns):
        raise ValueError("matmul_multi takes 1 to 4 handles and one N per handle")
    a = a2d.to(torch.float32).contiguous()
    M = a.shape[0]
    outs = [torch.empty((M, int(n)), dtype=torch.float32, device=a.device) for n in Ns]
    hv = (ctypes.c_void_p * len(handles))(*[int(h) for h in handles])
    cv = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
    _check_rc(_lib.i4_matmul_multi_dev(hv, len(handles), _vp(a.data_ptr()), int(M), cv, _torch_stream(a)),
              "i4_matmul_multi_dev")
    return outs


def rmsnorm_matmul_multi(x2d, w, eps, handles, Ns, want_hn=False):
    """GPU torch tensors x [M, K], w [K] -> [hn @ W_i for each handle], and hn
    when want_hn, with hn = rmsnorm(x, w, eps): the decoder's norm and the
    projections that read it (kernel/qwen35_decoder.cpp:279, 285-288), in
    one launch when the decode kernel quantizes the activation itself;
    asynchronous on the current stream."""
    _require_lib()
    import torch
    if not 1 <= len(handles) <= 4 or len(handles) != len(Ns):
        raise ValueError("rmsnorm_matmul_multi takes 1 to 4 handles and one N per handle")
    x = x2d.to(torch.float32).contiguous()
    M, K = x.shape
    wv = w.to(device=x.device, dtype=torch.float32).contiguous()
    if wv.numel() != K:
        raise ValueError(f"w has {wv.numel()} elements, x rows have {K}")
    outs = [torch.empty((M, int(n)), dtype=torch.float32, device=x.device) for n in Ns]
    hn = torch.empty_like(x) if want_hn else None
    hv = (ctypes.c_void_p * len(handles))(*[int(h) for h in handles])
    cv = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
    _check_rc(_lib.i4_rmsnorm_matmul_multi_dev(_vp(x.data_ptr()), _vp(wv.data_ptr()), float(eps), hv, len(handles),
                                               int(M), cv, _vp(hn.data_ptr()) if want_hn else None,
                                               _torch_stream(x)), "i4_rmsnorm_matmul_multi_dev")
    return (outs, hn) if want_hn else outs


def rmsnorm(x2d, w, eps):
    """GPU torch tensors x [s, H], w [H] -> fp32 [s, H]: the decoder's RMSNorm
    (kernel/qwen35_decoder.cpp:134-140) bit for bit, asynchronous on the
    current stream.  Its output is the activation of the projections that
    follow (input_ln / post_ln ahead of qkv, gate/up)."""
    _require_lib()
    import torch
    x = x2d.to(torch.float32).contiguous()
    if x.dim() != 2:
        raise ValueError(f"x must be 2-D [s, H], got shape {tuple(x.shape)}")
    s, H = x.shape
    wv = w.to(device=x.device, dtype=torch.float32).contiguous()
    if wv.numel() != H:
        raise ValueError(f"w has {wv.numel()} elements, x rows have {H}")
    out = torch.empty_like(x)
    if s == 0:
        return out
    _check_rc(_lib.i4_rmsnorm_dev(_vp(x.data_ptr()), _vp(wv.data_ptr()), int(s), int(H), float(eps),
                                  _vp(out.data_ptr()), _torch_stream(x)), "i4_rmsnorm_dev")
    return out


def matmul_argmax(handle, a2d, N):
    """GPU torch tensor [M, K] -> (logits fp32 [M, N], argmax int64 [M])."""
    _require_lib()
    import torch
    a = a2d.to(torch.float32).contiguous()
    M = a.shape[0]
    out = torch.empty((M, N), dtype=torch.float32, device=a.device)
    idx = torch.empty((M,), dtype=torch.int64, device=a.device)
    _check_rc(_lib.i4_matmul_argmax_dev(_vp(handle), _vp(a.data_ptr()), int(M), _vp(out.data_ptr()),
                                        _vp(idx.data_ptr()), _torch_stream(a)), "i4_matmul_argmax_dev")
    return out, idx


def block_dots(handle, a2d, N, K):
    """GPU torch tensor [M, K] -> int32 [M, N, K/32] exact block integers."""
    _require_lib()
    import torch
    a = a2d.to(torch.float32).contiguous()
    M = a.shape[0]
    cs = torch.empty((M, N, K // 32), dtype=torch.int32, device=a.device)
    _check_rc(_lib.i4_block_dots_dev(_vp(handle), _vp(a.data_ptr()), int(M), _vp(cs.data_ptr()),
                                     _torch_stream(a)), "i4_block_dots_dev")
    return cs


def handle_info(handle):
    _require_lib()
    out = np.zeros(8, np.int64)
    _check_rc(_lib.i4_handle_info(_vp(handle), _p(out)), "i4_handle_info")
    keys = ("N", "K", "bits", "scale_group", "has_zero_points", "has_corr_delta", "device_bytes",
            "device")
    return {k: int(v) for k, v in zip(keys, out)}


def unpack(handle):
    """Read a handle back as MatMulNBits arrays (qweight, scales, zp, corr_delta)."""
    info = handle_info(handle)
    N, K, bits = info["N"], info["K"], info["bits"]
    nblk = K // 32
    qw = np.empty((N, nblk, 4 * bits), np.uint8)
    sc = np.empty((N, nblk), np.float32)
    zp = np.empty((N, nblk), np.uint8)
    dl = np.empty((N, nblk), np.int32)
    _check_rc(_lib.i4_unpack(_vp(handle), _p(qw), _p(sc), _p(zp), _p(dl)), "i4_unpack")
    return dict(qweight=qw, scales=sc, zp=zp, corr_delta=dl, bits=bits)


def free(handle):
    if _lib is not None and handle:
        _lib.i4_free(_vp(handle))
