"""Python host binding of libspconv_amd.so (the C ABI declared in include/spconv_amd.h), over ctypes.

PyTorch is used only for device memory and the stream; every computation runs in the HIP library. There is no
CPU or PyTorch fallback: if the library is missing, loading raises.

Mirrors the reference's C++ operator interface (suvadityamuk/trellis2-cuda src/spconv.h:5-16):
    build_neighbors(coords, W, H, D) -> SpConvCache    (src/spconv.cu:38-54)
    SpConvCache.valid(B1) -> (list, seg)               (src/spconv.cu:56-75)
    spconv_cfg(N, Ci, Co) -> (B1, BK, S)               (src/spconv.cu:177-221)
    subm_conv(x, w, b, cache) -> y                     (src/spconv.cu:159-175)
plus subm_conv_fused (bias + SiLU / residual epilogue) and subdivide (src/sdec.cu:20-57).
Errors raise RuntimeError carrying spc_last_error() (the reference's t2_last_error convention, apps/t2lib.cu:23).
"""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG, "libspconv_amd.so")

F32, F16, BF16 = 0, 1, 2
ACT_NONE, ACT_SILU = 0, 1
EPI_F16_COMPAT = 256  # or'ed into act: the reference's fp16 epilogue rounding sequence
EMPTY = 0xFFFFFFFF

# the C ABI's exported symbols (every declaration of include/spconv_amd.h)
SYMBOLS = ("spc_last_error", "spc_set_stream", "spc_build_neighbors", "spc_build_neighbors_ex", "spc_cache_lookup",
           "spc_fdg_quads", "spc_cache_free", "spc_cache_info", "spc_cache_valid", "spc_conv_cfg",
           "spc_conv_cfg_autotune", "spc_conv_cfg_autotune_strict", "spc_subm_conv", "spc_subm_conv_fused", "spc_subm_conv_gathered",
           "spc_gather_ln_act", "spc_add_skip", "spc_convnext_mlp", "spc_subm_conv_skip",
           "spc_subdivide", "spc_subdivide_noalloc", "spc_subm_conv_replay", "spc_grid_sample_map",
           "spc_grid_sample_sum", "spc_subdivide_build", "spc_subm_conv_preln", "spc_alloc_counts", "spc_kernel_timing",
           "spc_kernel_times", "spc_release_cached_memory")

_lib = None


def load_library():
    """Load (once) and prototype the C ABI. Raises OSError if the library has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise OSError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() (make -C trellis2-cuda_amd)")
    L = ctypes.CDLL(LIB_PATH)
    P, I, I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    PP = ctypes.POINTER(ctypes.c_void_p)
    L.spc_last_error.restype = ctypes.c_char_p
    L.spc_last_error.argtypes = []
    L.spc_set_stream.argtypes = [P]
    L.spc_build_neighbors.argtypes = [P, I64, I, I, I, PP]
    L.spc_build_neighbors_ex.argtypes = [P, I64, I, I, I, I, PP]
    L.spc_cache_lookup.argtypes = [P, P, I64, P]
    L.spc_fdg_quads.argtypes = [P, P, P, P]
    L.spc_cache_free.argtypes = [P]
    L.spc_cache_info.argtypes = [P, ctypes.POINTER(I64), PP, PP, PP]
    L.spc_cache_valid.argtypes = [P, I, PP, PP, ctypes.POINTER(I64)]
    L.spc_conv_cfg.argtypes = [I64, I, I, ctypes.POINTER(I), ctypes.POINTER(I), ctypes.POINTER(I)]
    L.spc_conv_cfg_autotune.argtypes = [ctypes.c_char_p, ctypes.c_char_p, I64, I, I, ctypes.POINTER(I),
                                         ctypes.POINTER(I), ctypes.POINTER(I)]
    L.spc_conv_cfg_autotune_strict.argtypes = [ctypes.c_char_p, ctypes.c_char_p, I64, I, I, I, ctypes.POINTER(I),
                                                ctypes.POINTER(I), ctypes.POINTER(I)]
    L.spc_subm_conv.argtypes = [P, P, P, I, I, I64, I, I, P, P]
    L.spc_subm_conv_fused.argtypes = [P, P, P, P, I, I, I, I, I, I64, I, I, P, P]
    L.spc_subm_conv_gathered.argtypes = [P, I64, P, I, P, P, P, I, I, I, I, I, I64, I, I, P, P]
    L.spc_gather_ln_act.argtypes = [P, I64, I, P, I, P, P, ctypes.c_float, I, I, I64, P]
    L.spc_add_skip.argtypes = [P, P, P, I64, I, I64, I, I]
    L.spc_convnext_mlp.argtypes = [P, P, P, P, ctypes.c_float, P, P, P, P, I, I, I64, I, P]
    L.spc_subm_conv_skip.argtypes = [P, P, P, I, I, I, P, I64, I, P, I64, I, I, P, P]
    L.spc_subdivide.argtypes = [P, P, I64, P, P, ctypes.POINTER(I64)]
    L.spc_subdivide_noalloc.argtypes = [P, P, I64, P, P, P]
    L.spc_subm_conv_replay.argtypes = [P, P, P, P, I, I64, I, I, I, I, I, P, P]
    L.spc_grid_sample_map.argtypes = [P, P, I64, I, I, P, P]
    L.spc_grid_sample_sum.argtypes = [P, I64, I, P, P, I64, P]
    L.spc_subdivide_build.argtypes = [P, P, I64, I, I, I, P, P, ctypes.POINTER(I64), PP]
    L.spc_subm_conv_preln.argtypes = [P, I64, P, I, P, P, ctypes.c_float, I, P, P, I, I, I, P, I64, I, P, I64, I, I,
                                      P, P]
    L.spc_alloc_counts.argtypes = [ctypes.POINTER(I64), ctypes.POINTER(I64)]
    L.spc_kernel_timing.argtypes = [I]
    L.spc_release_cached_memory.argtypes = [ctypes.POINTER(I64)]
    L.spc_kernel_times.argtypes = [ctypes.POINTER(ctypes.c_float), I, ctypes.POINTER(I)]
    for name in SYMBOLS:
        if name != "spc_last_error":
            getattr(L, name).restype = I
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(load_library().spc_last_error().decode(errors="replace"))


def _torch():
    import torch
    return torch


def _dt(t) -> int:
    torch = _torch()
    m = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
    if t.dtype not in m:
        raise TypeError(f"unsupported dtype {t.dtype}")
    return m[t.dtype]


def _ptr(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("tensor must be on the GPU")
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


def set_stream(stream=None) -> None:
    """Run later calls on a torch.cuda.Stream (None = torch's current stream)."""
    torch = _torch()
    s = torch.cuda.current_stream() if stream is None else stream
    _check(load_library().spc_set_stream(ctypes.c_void_p(s.cuda_stream)))


class SpConvCache:
    """Owns one neighbour cache (nbr/gray/sorted + memoized valid lists); freed on garbage collection."""

    def __init__(self, handle, n, device):
        self._h = handle
        self.N = n
        self.device = device

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.spc_cache_free(self._h)
            self._h = None

    def _view(self, ptr, shape, dtype):
        torch = _torch()
        numel = 1
        for s in shape:
            numel *= s
        if numel == 0:
            return torch.empty(shape, dtype=dtype, device=self.device)
        # copy out of the library-owned buffer (the cache keeps ownership)
        out = torch.empty(shape, dtype=dtype, device=self.device)
        _memcpy_d2d(out.data_ptr(), ptr, out.numel() * out.element_size())
        return out

    def tensors(self):
        """(nbr int32 [N,27] with -1 = EMPTY, gray int32 [N], sorted int32 [N]) as new torch tensors."""
        torch = _torch()
        n = ctypes.c_int64()
        nbr, gray, srt = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        _check(load_library().spc_cache_info(self._h, ctypes.byref(n), ctypes.byref(nbr), ctypes.byref(gray),
                                             ctypes.byref(srt)))
        N = n.value
        return (self._view(nbr.value, (N, 27), torch.int32), self._view(gray.value, (N,), torch.int32),
                self._view(srt.value, (N,), torch.int32))

    def valid(self, B1: int):
        """(list int32 [L], seg int32 [ceil(N/B1)+1]) as new torch tensors."""
        torch = _torch()
        lst, seg, L = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_int64()
        _check(load_library().spc_cache_valid(self._h, B1, ctypes.byref(lst), ctypes.byref(seg), ctypes.byref(L)))
        nb = (self.N + B1 - 1) // B1
        return self._view(lst.value, (L.value,), torch.int32), self._view(seg.value, (nb + 1,), torch.int32)


_hip = None


def _memcpy_d2d(dst: int, src: int, nbytes: int) -> None:
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _hip.hipMemcpy.restype = ctypes.c_int
        _hip.hipDeviceSynchronize.restype = ctypes.c_int
    _hip.hipDeviceSynchronize()  # the library may run on a stream other than torch's
    rc = _hip.hipMemcpy(ctypes.c_void_p(dst), ctypes.c_void_p(src), ctypes.c_size_t(nbytes), 3)
    if rc != 0:
        raise RuntimeError(f"hipMemcpy failed ({rc})")


def build_neighbors(coords, W: int = 4096, H: int = 4096, D: int = 4096, keep_hash: bool = False) -> SpConvCache:
    """Kernel map of coords (int32 [N,4] = (b,x,y,z)) in a W x H x D grid (reference build_neighbors,
    src/spconv.cu:38-54). keep_hash keeps the voxel hash for lookup()."""
    torch = _torch()
    if coords.dtype != torch.int32 or coords.dim() != 2 or coords.shape[1] != 4:
        raise ValueError("coords must be int32 [N,4]")
    h = ctypes.c_void_p()
    _check(load_library().spc_build_neighbors_ex(_ptr(coords), coords.shape[0], W, H, D, 1 if keep_hash else 0,
                                                 ctypes.byref(h)))
    return SpConvCache(h, coords.shape[0], coords.device)


def lookup(cache: SpConvCache, query):
    """Row of each (b,x,y,z) query (int32 [M,4]) in the cache's voxels, -1 when absent or outside the grid; the cache
    must be built with keep_hash (reference vhash_find, src/mesh.cu:14-19)."""
    torch = _torch()
    if query.dtype != torch.int32 or query.dim() != 2 or query.shape[1] != 4:
        raise ValueError("query must be int32 [M,4]")
    rows = torch.empty(query.shape[0], dtype=torch.int32, device=query.device)
    _check(load_library().spc_cache_lookup(cache._h, _ptr(query), query.shape[0], _ptr(rows)))
    return rows


def fdg_quads(cache: SpConvCache, h):
    """FlexiDualGrid quads from the kernel map (reference k_fdg_quads, src/mesh.cu:36-45): returns (quad int32
    [3N,4], ok int32 [3N]); quad rows of edges with ok = 0 are unspecified."""
    torch = _torch()
    if h.dtype != torch.float32 or h.dim() != 2 or h.shape != (cache.N, 7):
        raise ValueError(f"h must be float32 [{cache.N},7]")
    quad = torch.full((3 * cache.N, 4), -1, dtype=torch.int32, device=h.device)
    ok = torch.empty(3 * cache.N, dtype=torch.int32, device=h.device)
    _check(load_library().spc_fdg_quads(cache._h, _ptr(h), _ptr(quad), _ptr(ok)))
    return quad, ok


def grid_sample_map(cache: SpConvCache, grid, batch: int = 0, normalize: bool = False):
    """Trilinear sample map of points grid (float32 [L,3], continuous voxel coordinates) on a keep_hash cache:
    (nb int32 [L,8] rows or -1, wt float32 [L,8]); the bake's grid-sample map (src/glb.cu:547-550)."""
    torch = _torch()
    if grid.dtype != torch.float32 or grid.dim() != 2 or grid.shape[1] != 3:
        raise ValueError("grid must be float32 [L,3]")
    L = grid.shape[0]
    nb = torch.empty((L, 8), dtype=torch.int32, device=grid.device)
    wt = torch.empty((L, 8), dtype=torch.float32, device=grid.device)
    _check(load_library().spc_grid_sample_map(cache._h, _ptr(grid), L, batch, 1 if normalize else 0, _ptr(nb),
                                              _ptr(wt)))
    return nb, wt


def grid_sample_sum(x, nb, wt):
    """y float32 [L,C] = sum_v x[nb[:,v]] * wt[:,v] (reference k_wsum, src/glb.cu:456-465)."""
    torch = _torch()
    if x.dtype != torch.float32 or x.dim() != 2:
        raise ValueError("x must be float32 [M,C]")
    L, C = nb.shape[0], x.shape[1]
    y = torch.empty((L, C), dtype=torch.float32, device=x.device)
    _check(load_library().spc_grid_sample_sum(_ptr(x), x.shape[0], C, _ptr(nb), _ptr(wt), L, _ptr(y)))
    return y


def spconv_cfg(N: int, Ci: int, Co: int):
    b1, bk, s = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _check(load_library().spc_conv_cfg(N, Ci, Co, ctypes.byref(b1), ctypes.byref(bk), ctypes.byref(s)))
    return b1.value, bk.value, s.value


def spconv_cfg_autotune(path: str, device: str, N: int, Ci: int, Co: int, strict: bool = False):
    """(B1, BK, S) the reference would pick from a FlexGEMM autotune cache file for device section `device`
    (reference spconv_cfg, src/spconv.cu:176-221); (128, 64, 1) where the file has no entry, or RuntimeError when
    `strict` (or T2_STRICT=1 in the environment, src/spconv.cu:219). Host only."""
    b1, bk, s = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _check(load_library().spc_conv_cfg_autotune_strict(os.fsencode(path), device.encode(), N, Ci, Co, int(strict),
                                                       ctypes.byref(b1), ctypes.byref(bk), ctypes.byref(s)))
    return b1.value, bk.value, s.value


def subm_conv_fused(x, w, b, cache: SpConvCache, residual=None, act: int = ACT_NONE, out=None, out_dtype=None):
    """out = act(subm_conv3d(x, w) + b) [+ residual]; w is [Co,27,Ci] (= torch [Co,3,3,3,Ci].view)."""
    torch = _torch()
    N, Ci = x.shape
    Co = w.shape[0]
    if w.dtype != x.dtype:  # the C ABI carries one dtype code for x and w
        raise ValueError(f"x and w must both be bf16 or both fp16 (x {x.dtype}, w {w.dtype})")
    if out is None:
        out = torch.empty((N, Co), dtype=out_dtype or x.dtype, device=x.device)
    _check(load_library().spc_subm_conv_fused(
        _ptr(x), _ptr(w), _ptr(b), _ptr(residual), _dt(x), _dt(b) if b is not None else F32,
        _dt(residual) if residual is not None else F32, _dt(out), act, N, Ci, Co, cache._h, _ptr(out)))
    return out


def subm_conv_gathered(x_src, row_map, shift: int, w, b, cache: SpConvCache, residual=None, act: int = ACT_NONE,
                       out=None, out_dtype=None):
    """subm_conv_fused on x = x_src[row_map >> shift] without materializing it (e.g. c2s children reading their
    parents' rows: row_map = src, shift = 3). Map entries outside [0, len(x_src)) read zero rows."""
    torch = _torch()
    M, Ci = x_src.shape
    N = cache.N
    Co = w.shape[0]
    if w.dtype != x_src.dtype:
        raise ValueError(f"x_src and w must both be bf16 or both fp16 (x {x_src.dtype}, w {w.dtype})")
    if row_map.dtype != torch.int32 or row_map.numel() != N:
        raise ValueError(f"row_map must be int32 [{N}]")
    if out is None:
        out = torch.empty((N, Co), dtype=out_dtype or x_src.dtype, device=x_src.device)
    _check(load_library().spc_subm_conv_gathered(
        _ptr(x_src), M, _ptr(row_map), shift, _ptr(w), _ptr(b), _ptr(residual), _dt(x_src),
        _dt(b) if b is not None else F32, _dt(residual) if residual is not None else F32, _dt(out), act, N, Ci, Co,
        cache._h, _ptr(out)))
    return out


def gather_ln_act(x_src, row_map=None, shift: int = 0, gamma=None, beta=None, eps: float = 1e-6,
                  act: int = ACT_SILU, out=None):
    """act(LayerNorm(x_src[row_map >> shift]) * gamma + beta) in one pass, fp32 statistics, one rounding to
    x_src's dtype (reference layer_norm + act_ SILU, src/ops.cu:30-75, and the upsample block's gather before them,
    src/sdec.cu:78-83). row_map None: the rows of x_src in order. Map entries outside [0, len(x_src)) read zero
    rows."""
    torch = _torch()
    M, C = x_src.shape
    if row_map is not None and (row_map.dtype != torch.int32 or row_map.dim() != 1):
        raise ValueError("row_map must be int32 [N]")
    N = M if row_map is None else row_map.numel()
    for name, t in (("gamma", gamma), ("beta", beta)):
        if t is not None and (t.dtype != torch.float32 or t.numel() != C):
            raise ValueError(f"{name} must be float32 [{C}]")
    if out is None:
        out = torch.empty((N, C), dtype=x_src.dtype, device=x_src.device)
    _check(load_library().spc_gather_ln_act(_ptr(x_src), M, C, _ptr(row_map), shift, _ptr(gamma), _ptr(beta),
                                            eps, act, _dt(x_src), N, _ptr(out)))
    return out


def convnext_mlp(h, x, gamma, beta, w1, b1, w2, b2, eps: float = 1e-6, out=None):
    """x + W2 silu(W1 (LayerNorm(h) * gamma + beta) + b1) + b2 in one pass (the tail of the reference's
    SDecoder::convnext after its conv, src/sdec.cu:60-66). w1 [4C, C], w2 [C, 4C] in h's dtype; gamma, beta, b1, b2
    share one float dtype (or are None). out may be h or x."""
    N, C = h.shape
    ps = [p for p in (gamma, beta, b1, b2) if p is not None]
    if any(p.dtype != ps[0].dtype for p in ps):
        raise ValueError("gamma, beta, b1, b2 must share one dtype")
    for name, t in (("x", x), ("w1", w1), ("w2", w2)):
        if t.dtype != h.dtype:
            raise ValueError(f"{name} must have h's dtype {h.dtype}")
    if out is None:
        out = _torch().empty_like(h)
    _check(load_library().spc_convnext_mlp(_ptr(h), _ptr(x), _ptr(gamma), _ptr(beta), eps, _ptr(w1), _ptr(b1),
                                           _ptr(w2), _ptr(b2), _dt(h), _dt(ps[0]) if ps else F32, N, C,
                                           _ptr(out)))
    return out


def subm_conv_skip(x, w, b, cache: SpConvCache, x_skip, src, act: int = ACT_NONE, out=None):
    """act(subm_conv3d(x, w) + b) + repeat_interleave(C2S(x_skip), Co / (Cin/8), dim=1) in one pass (the reference's
    conv2 + k_add_skip of SDecoder::up, src/sdec.cu:38-43, 82-84); out has x's 16-bit dtype."""
    torch = _torch()
    N, Ci = x.shape
    Co = w.shape[0]
    n_skip, Cin = x_skip.shape
    if src.dtype != torch.int32 or src.numel() != N:
        raise ValueError(f"src must be int32 [{N}]")
    if out is None:
        out = torch.empty((N, Co), dtype=x.dtype, device=x.device)
    _check(load_library().spc_subm_conv_skip(_ptr(x), _ptr(w), _ptr(b), _dt(x), _dt(b) if b is not None else F32, act,
                                             _ptr(x_skip), n_skip, Cin, _ptr(src), N, Ci, Co, cache._h, _ptr(out)))
    return out


def subm_conv_preln(x_src, w, b, cache: SpConvCache, row_map=None, shift: int = 0, gamma=None, beta=None,
                    eps: float = 1e-6, pre_act: int = ACT_SILU, act: int = ACT_NONE, x_skip=None, skip_src=None,
                    out=None):
    """act(subm_conv3d(pre_act(LayerNorm(x_src[row_map >> shift]) * gamma + beta), w) + b) [+ the skip of
    subm_conv_skip when x_skip / skip_src are given]: the upsample block's norm2 + SiLU + conv2 + skip
    (src/sdec.cu:78-84). gather_ln_act then the conv; with SPCONV_PRELN_FUSED=1 in the environment, one kernel for
    64 -> 64 convs whose halo schedule has no spill tiles; the same bits either way. out has x_src's 16-bit
    dtype."""
    torch = _torch()
    M, Ci = x_src.shape
    Co = w.shape[0]
    N = cache.N
    if row_map is not None and (row_map.dtype != torch.int32 or row_map.numel() != N):
        raise ValueError(f"row_map must be int32 [{N}]")
    for name, t in (("gamma", gamma), ("beta", beta)):
        if t is not None and (t.dtype != torch.float32 or t.numel() != Ci):
            raise ValueError(f"{name} must be float32 [{Ci}]")
    if (x_skip is None) != (skip_src is None):
        raise ValueError("x_skip and skip_src go together")
    if skip_src is not None and (skip_src.dtype != torch.int32 or skip_src.numel() != N):
        raise ValueError(f"skip_src must be int32 [{N}]")
    n_skip, Cin = x_skip.shape if x_skip is not None else (0, 0)
    if out is None:
        out = torch.empty((N, Co), dtype=x_src.dtype, device=x_src.device)
    _check(load_library().spc_subm_conv_preln(
        _ptr(x_src), M, _ptr(row_map), shift, _ptr(gamma), _ptr(beta), eps, pre_act, _ptr(w), _ptr(b), _dt(x_src),
        _dt(b) if b is not None else F32, act, _ptr(x_skip), n_skip, Cin, _ptr(skip_src), N, Ci, Co, cache._h,
        _ptr(out)))
    return out


def add_skip(h, x, src):
    """In place: h += repeat_interleave(C2S(x), Co / (Cin/8), dim=1), i.e. child row i, channel c gets
    x[src[i] >> 3, (src[i] & 7) * Cin/8 + c // rep] (reference k_add_skip, src/sdec.cu:38-43); returns h."""
    torch = _torch()
    m, Co = h.shape
    n, Cin = x.shape
    if h.dtype != x.dtype:
        raise ValueError(f"h and x must share a dtype ({h.dtype}, {x.dtype})")
    if src.dtype != torch.int32 or src.numel() != m:
        raise ValueError(f"src must be int32 [{m}]")
    _check(load_library().spc_add_skip(_ptr(h), _ptr(x), _ptr(src), m, Co, n, Cin, _dt(h)))
    return h


def subm_conv(x, w, b, cache: SpConvCache):
    """y = subm_conv3d(x, w, b) in x's dtype (reference subm_conv, src/spconv.cu:159-175)."""
    torch = _torch()
    N, Ci = x.shape
    Co = w.shape[0]
    if w.dtype != x.dtype:
        raise ValueError(f"x and w must both be bf16 or both fp16 (x {x.dtype}, w {w.dtype})")
    y = torch.empty((N, Co), dtype=x.dtype, device=x.device)
    _check(load_library().spc_subm_conv(_ptr(x), _ptr(w), _ptr(b), _dt(x), _dt(b) if b is not None else F32,
                                        N, Ci, Co, cache._h, _ptr(y)))
    return y


def subm_conv_replay(x, w, b, cache, cfg, residual=None, act=ACT_NONE):
    """The reference's fp16 conv under the tile choice cfg = (B1, BK, S), rounding included (split-K partials summed
    with four interleaved accumulators when S > 1). fp16 x, w, b, residual; returns fp16 [N, Co]."""
    torch = _torch()
    N, Ci = x.shape
    Co = w.shape[0]
    y = torch.empty((N, Co), dtype=torch.float16, device=x.device)
    B1, BK, S = cfg
    _check(load_library().spc_subm_conv_replay(_ptr(x), _ptr(w), _ptr(b), _ptr(residual), act, N, Ci, Co, B1, BK, S,
                                               cache._h, _ptr(y)))
    return y


def subdivide(coords, logits_f16):
    """(child coords int32 [M,4], src int32 [M]) for children whose fp16 logit is > 0."""
    torch = _torch()
    n = coords.shape[0]
    cc = torch.empty((max(8 * n, 1), 4), dtype=torch.int32, device=coords.device)
    src = torch.empty((max(8 * n, 1),), dtype=torch.int32, device=coords.device)
    m = ctypes.c_int64()
    _check(load_library().spc_subdivide(_ptr(coords), _ptr(logits_f16), n, _ptr(cc), _ptr(src), ctypes.byref(m)))
    return cc[:m.value], src[:m.value]


def kernel_timing(on: bool):
    """Start (clearing earlier records) or stop bracketing each conv call's conv kernels with HIP events on the
    library stream (the weight repack and first-call schedules fall outside)."""
    _check(load_library().spc_kernel_timing(int(on)))


def kernel_times():
    """Per-call conv-kernel times (ms) recorded since kernel_timing(True), in call order (waits for them)."""
    L = load_library()
    n = ctypes.c_int()
    _check(L.spc_kernel_times(None, 0, ctypes.byref(n)))
    buf = (ctypes.c_float * max(n.value, 1))()
    _check(L.spc_kernel_times(buf, n.value, ctypes.byref(n)))
    return list(buf[:n.value])


def release_cached_memory() -> int:
    """Return the library's cached, unused device blocks to the driver; the bytes released."""
    b = ctypes.c_int64()
    _check(load_library().spc_release_cached_memory(ctypes.byref(b)))
    return b.value


def alloc_counts():
    """(allocation requests, hipMallocAsync calls) the library has made in this process (host only)."""
    r, d = ctypes.c_int64(), ctypes.c_int64()
    _check(load_library().spc_alloc_counts(ctypes.byref(r), ctypes.byref(d)))
    return r.value, d.value


def subdivide_build(coords, logits_f16, W: int = 4096, H: int = 4096, D: int = 4096):
    """(child coords int32 [M,4], src int32 [M], SpConvCache of the children) with no host sync between the
    subdivision and the map build (reference SDecoder::c2s, src/sdec.cu:45-56)."""
    torch = _torch()
    n = coords.shape[0]
    cc = torch.empty((max(8 * n, 1), 4), dtype=torch.int32, device=coords.device)
    src = torch.empty((max(8 * n, 1),), dtype=torch.int32, device=coords.device)
    m = ctypes.c_int64()
    h = ctypes.c_void_p()
    _check(load_library().spc_subdivide_build(_ptr(coords), _ptr(logits_f16), n, W, H, D, _ptr(cc), _ptr(src),
                                              ctypes.byref(m), ctypes.byref(h)))
    return cc[:m.value], src[:m.value], SpConvCache(h, m.value, coords.device)


def source_digest() -> str:
    """sha256 over the HIP/C++ sources of the library (file names and contents, sorted): stamps measured profile
    figures with the code they were measured on, so a stale figure can be recognised."""
    import hashlib
    d = os.path.join(_PKG, "csrc")
    h = hashlib.sha256()
    for name in sorted(os.listdir(d)):
        if name.endswith((".hip", ".h")):
            h.update(name.encode())
            with open(os.path.join(d, name), "rb") as f:
                h.update(f.read())
    return h.hexdigest()[:16]
