"""Tensor-level front end of libwave_runtime.so.

PyTorch only provides device memory and the current stream here; all
arithmetic runs in the library's gfx950 kernels.  Argument errors raise
ValueError (as the reference's builders do, wave_matmul.py:533-775) and HIP
failures raise runtime.WaveError.
"""

from __future__ import annotations

import ctypes

import torch

from . import runtime as rt

_DT = {torch.float32: rt.F32, torch.float16: rt.F16, torch.bfloat16: rt.BF16}
_NAMES = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _dtype(d) -> torch.dtype:
    return _NAMES[d] if isinstance(d, str) else d


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _need(t: torch.Tensor, name: str, device: torch.device | None = None) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, not {device}")


def _out(out: torch.Tensor | None, shape, dtype: torch.dtype, device: torch.device,
         name: str = "out") -> torch.Tensor:
    """A caller's output tensor checked for shape, dtype, device and
    contiguity (the kernels write exactly that many elements through a bare
    pointer), or a new one."""
    if out is None:
        return torch.empty(shape, dtype=dtype, device=device)
    if tuple(out.shape) != tuple(shape) or out.dtype != dtype:
        raise ValueError(f"{name} must be {dtype} {tuple(shape)}, got {out.dtype} "
                         f"{tuple(out.shape)}")
    _need(out, name, device)
    return out


def gemm(a: torch.Tensor, b: torch.Tensor, *, out_dtype="f16",
         layout: str = "row", out: torch.Tensor | None = None) -> torch.Tensor:
    """C = A . B^T with A [M, K] and B [N, K] (f16 or bf16), fp32 accumulate.

    layout "row" returns C as [M, N]; "col" returns the column-major buffer
    viewed as [N, M] (element (n, m) = C[m, n]).
    """
    M, N, K = _gemm_operands(a, b)
    if layout not in ("row", "col"):
        raise ValueError("layout must be 'row' or 'col'")
    odt = _dtype(out_dtype)
    out = _out(out, (M, N) if layout == "row" else (N, M), odt, a.device)
    rt.check(rt.lib().wave_gemm_launch(
        a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K, _DT[a.dtype], _DT[odt],
        rt.ROW_MAJOR if layout == "row" else rt.COL_MAJOR, _stream(a)))
    return out


def _gemm_operands(a: torch.Tensor, b: torch.Tensor) -> tuple[int, int, int]:
    _need(a, "a")
    _need(b, "b", a.device)
    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[1]:
        raise ValueError("a must be [M, K] and b [N, K]")
    if a.dtype != b.dtype or a.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("a and b must both be f16 or both bf16")
    return a.shape[0], b.shape[0], a.shape[1]


def gemm_auto_workspace_bytes(M: int, N: int, K: int) -> int:
    n = ctypes.c_size_t()
    rt.check(rt.lib().wave_gemm_auto_workspace_bytes(M, N, K, ctypes.byref(n)))
    return n.value


def gemm_auto(a: torch.Tensor, b: torch.Tensor, *, out_dtype="f16", layout: str = "row",
              workspace: torch.Tensor | None = None,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """C = A . B^T through the shape-driven dispatch (wave_gemm_auto_launch):
    for M <= 128 the short-M kernel, split over K when its 128-column blocks
    would leave CUs idle; otherwise Stream-K when the 256x256 tiles would leave
    half the CUs idle, else the tiled kernel.  workspace: a device byte tensor of at least
    gemm_auto_workspace_bytes(M, N, K) bytes (allocated here when None)."""
    M, N, K = _gemm_operands(a, b)
    if layout not in ("row", "col"):
        raise ValueError("layout must be 'row' or 'col'")
    odt = _dtype(out_dtype)
    out = _out(out, (M, N) if layout == "row" else (N, M), odt, a.device)
    need = gemm_auto_workspace_bytes(M, N, K)
    if workspace is None and need:
        workspace = torch.empty(need, dtype=torch.uint8, device=a.device)
    if workspace is not None:
        _need(workspace, "workspace", a.device)
    rt.check(rt.lib().wave_gemm_auto_launch(
        a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K, _DT[a.dtype], _DT[odt],
        rt.ROW_MAJOR if layout == "row" else rt.COL_MAJOR,
        workspace.data_ptr() if workspace is not None else None,
        workspace.numel() * workspace.element_size() if workspace is not None else 0,
        _stream(a)))
    return out


def gemm_tile_packed(a: torch.Tensor, b: torch.Tensor, *, bm: int = 1, bn: int = 1,
                     wave_m_tiles: int = 1, wave_n_tiles: int = 1, out_dtype="f32",
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """C = A . B^T stored tile-packed (1-D, M*N elements) for the reference
    blocking (bm, bn, wave_m_tiles, wave_n_tiles): the reference's
    output_layout "tile-packed" (wave_gemm_tile_packed_launch)."""
    M, N, K = _gemm_operands(a, b)
    odt = _dtype(out_dtype)
    out = _out(out, (M * N,), odt, a.device)
    rt.check(rt.lib().wave_gemm_tile_packed_launch(
        a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K, _DT[a.dtype], _DT[odt], bm, bn,
        wave_m_tiles, wave_n_tiles, _stream(a)))
    return out


def gemm_mxfp4(a: torch.Tensor, b: torch.Tensor, a_scale: torch.Tensor,
               b_scale: torch.Tensor, *, out_dtype="f32", layout: str = "row",
               input_layout: str = "canonical",
               out: torch.Tensor | None = None) -> torch.Tensor:
    """MXFP4 scaled GEMM (the reference's ``mxfp4`` input type,
    wave_matmul.py:996-1022): A [M, K/2] and B [N, K/2] uint8, two e2m1
    values per byte (low nibble = even k); a_scale [K/32, M] and b_scale
    [K/32, N] uint8 e8m0.  C[m, n] = sum_k a[m, k] 2^(sa[k/32, m]-127) *
    b[n, k] 2^(sb[k/32, n]-127), fp32 accumulate.  layout as in gemm().

    input_layout "aiter": b [N, K/2] holds the AITER-preshuffled bytes and
    the scales are the AITER blocks (1-D, M*G8*8 and N*G8*8 bytes with G8 =
    ceil(K/256); wave_gemm_mxfp4_aiter_launch).
    """
    aiter = input_layout == "aiter"
    if input_layout not in ("canonical", "aiter"):
        raise ValueError("input_layout must be 'canonical' or 'aiter'")
    for t, name in ((a, "a"), (b, "b"), (a_scale, "a_scale"), (b_scale, "b_scale")):
        _need(t, name)
        if t.dtype != torch.uint8 or t.dim() != (1 if aiter and "scale" in name else 2):
            raise ValueError(f"{name} has the wrong dtype or rank")
    M, KB = a.shape
    N = b.shape[0]
    K = 2 * KB
    if b.shape[1] != KB:
        raise ValueError("a must be [M, K/2] and b [N, K/2]")
    if aiter:
        g8 = (K // 32 + 7) // 8
        if K % 32 or a_scale.numel() != M * g8 * 8 or b_scale.numel() != N * g8 * 8:
            raise ValueError("AITER scales must hold M*G8*8 and N*G8*8 bytes")
    elif K % 32 or tuple(a_scale.shape) != (K // 32, M) or tuple(b_scale.shape) != (K // 32, N):
        raise ValueError("scales must be [K/32, M] and [K/32, N]")
    for t, name in ((b, "b"), (a_scale, "a_scale"), (b_scale, "b_scale")):
        _need(t, name, a.device)
    if layout not in ("row", "col"):
        raise ValueError("layout must be 'row' or 'col'")
    odt = _dtype(out_dtype)
    out = _out(out, (M, N) if layout == "row" else (N, M), odt, a.device)
    fn = rt.lib().wave_gemm_mxfp4_aiter_launch if aiter else rt.lib().wave_gemm_mxfp4_launch
    rt.check(fn(a.data_ptr(), b.data_ptr(), out.data_ptr(), a_scale.data_ptr(),
                b_scale.data_ptr(), M, N, K, _DT[odt],
                rt.ROW_MAJOR if layout == "row" else rt.COL_MAJOR, _stream(a)))
    return out


def streamk_workspace_bytes(M: int, N: int, workers: int) -> tuple[int, int]:
    s, c = ctypes.c_size_t(), ctypes.c_size_t()
    rt.check(rt.lib().wave_gemm_streamk_workspace_bytes(M, N, workers, ctypes.byref(s),
                                                        ctypes.byref(c)))
    return s.value, c.value


class StreamKWorkspace:
    """Caller-owned Stream-K workspace: fp32 partial slots + zeroed counters."""

    def __init__(self, M: int, N: int, workers: int, device="cuda"):
        sb, cb = streamk_workspace_bytes(M, N, workers)
        self.M, self.N, self.workers = M, N, workers
        self.scratch = torch.empty(sb // 4, dtype=torch.float32, device=device)
        self.counters = torch.zeros(cb // 4, dtype=torch.int32, device=device)

    def reset(self) -> None:
        rt.check(rt.lib().wave_gemm_streamk_workspace_reset(
            self.counters.data_ptr(), self.M, self.N, _stream(self.counters)))

    def nonzero_counters(self) -> int:
        r = rt.lib().wave_gemm_streamk_counters_check(
            self.counters.data_ptr(), self.M, self.N, _stream(self.counters))
        if r < 0 or r > self.counters.numel():
            rt.check(r)
        return r


def gemm_streamk(a: torch.Tensor, b: torch.Tensor, workers: int, *,
                 out_dtype="f16", layout: str = "row",
                 workspace: StreamKWorkspace | None = None,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """Stream-K C = A . B^T over `workers` persistent workgroups.

    A caller's workspace must have been made for this (M, N) and at least
    `workers` workers, on a's device: the kernels index its partial slots
    and counters through bare pointers."""
    M, N, K = _gemm_operands(a, b)
    if layout not in ("row", "col"):
        raise ValueError("layout must be 'row' or 'col'")
    odt = _dtype(out_dtype)
    out = _out(out, (M, N) if layout == "row" else (N, M), odt, a.device)
    if workspace is not None:
        if workspace.M != M or workspace.N != N or workspace.workers < workers:
            raise ValueError(f"workspace is for M={workspace.M} N={workspace.N} "
                             f"workers={workspace.workers}, not M={M} N={N} workers={workers}")
        _need(workspace.scratch, "workspace.scratch", a.device)
        _need(workspace.counters, "workspace.counters", a.device)
    ws = workspace or StreamKWorkspace(M, N, workers, a.device)
    rt.check(rt.lib().wave_gemm_streamk_launch(
        a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K, _DT[a.dtype], _DT[odt],
        rt.ROW_MAJOR if layout == "row" else rt.COL_MAJOR, ws.scratch.data_ptr(),
        ws.counters.data_ptr(), workers, _stream(a)))
    return out


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                    causal: bool = False, scale: float | None = None,
                    qk_max_abs: float | None = None, waves: int = 8,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """softmax(Q K^T * scale) V for q [B, Hq, S, D], k/v [B, Hkv, S, D].

    qk_max_abs: the caller's bound on |Q| and |K|; selects the fixed-max
    kernel (no online max; wave_fa_fwd_bounded_launch).  waves: 8 (the
    ping-pong kernel), 12 (three rotating wave groups, 384 query rows a
    CTA) or 4 (the reference's 4-wave configuration); other than 8 through
    wave_fa_fwd_config_launch."""
    B, Hq, Hkv, S, D = _fa_shapes(q, k, v)
    out = _out(out, q.shape, q.dtype, q.device)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, Hq, Hkv, S, D,
            _DT[q.dtype], int(causal), float(scale or 0.0))
    if waves != 8:
        rt.check(rt.lib().wave_fa_fwd_config_launch(
            *args, 0.0 if qk_max_abs is None else float(qk_max_abs), int(waves),
            _stream(q)))
    elif qk_max_abs is None:
        rt.check(rt.lib().wave_fa_fwd_launch(*args, _stream(q)))
    else:
        rt.check(rt.lib().wave_fa_fwd_bounded_launch(*args, float(qk_max_abs), _stream(q)))
    return out


def _fa_shapes(q, k, v):
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _need(t, n, q.device)
        if t.dim() != 4:
            raise ValueError(f"{n} must be [batch, heads, seq, head_dim]")
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("q, k, v must share an f16 or bf16 dtype")
    B, Hq, S, D = q.shape
    if k.shape != v.shape or k.shape[0] != B or k.shape[2] != S or k.shape[3] != D:
        raise ValueError("k and v must be [batch, kv_heads, seq, head_dim]")
    return B, Hq, k.shape[1], S, D


def mxfp8_quantize(x: torch.Tensor, dim: int = -1) -> tuple[torch.Tensor, torch.Tensor]:
    """OCP MX-FP8 encoding of x along `dim` (its size a multiple of 32, or
    padded with zeros to one): blocks of 32 elements share the e8m0 scale
    2^(floor(log2(amax)) - 8) (the OCP MX rule for e4m3, whose largest
    exponent is 8), and each element is x / scale rounded to e4m3, saturated at
    +-448.  Returns (e4m3 bytes as uint8, x's shape; e8m0 bytes as uint8, x's
    shape with `dim` divided by 32, rounded up)."""
    dim = dim % x.dim()
    xs = x.float().movedim(dim, -1)
    n = xs.shape[-1]
    nb = -(-n // 32)
    if nb * 32 != n:
        xs = torch.nn.functional.pad(xs, (0, nb * 32 - n))
    blocks = xs.reshape(*xs.shape[:-1], nb, 32)
    amax = blocks.abs().amax(dim=-1)
    e = torch.where(amax > 0, torch.floor(torch.log2(amax)) - 8, torch.full_like(amax, -127))
    e = e.clamp(-127, 127)
    q = (blocks / torch.exp2(e).unsqueeze(-1)).clamp(-448.0, 448.0)
    elems = q.to(torch.float8_e4m3fn).view(torch.uint8).reshape(*xs.shape)[..., :n]
    scales = (e + 127).to(torch.uint8)
    return elems.movedim(-1, dim).contiguous(), scales.movedim(-1, dim).contiguous()


def flash_attention_mxfp8(q: torch.Tensor, q_scale: torch.Tensor, k: torch.Tensor,
                          k_scale: torch.Tensor, v: torch.Tensor, v_scale: torch.Tensor, *,
                          causal: bool = False, scale: float | None = None, out_dtype="f16",
                          out: torch.Tensor | None = None, lse: torch.Tensor | None = None
                          ) -> torch.Tensor:
    """softmax(Q K^T * scale) V of block-scaled FP8 inputs
    (wave_fa_fwd_mxfp8_launch): q [B, Hq, S, 128], k / v [B, Hkv, S, 128]
    e4m3 bytes (uint8 or float8_e4m3fn); q_scale [B, Hq, S, 4], k_scale
    [B, Hkv, S, 4] and v_scale [B, Hkv, ceil(S/32), 128] e8m0 bytes, as
    mxfp8_quantize(q), mxfp8_quantize(k) and mxfp8_quantize(v, dim=2) return
    them.  lse: an optional float32 [B, Hq, S] output."""
    def raw(t, name):
        _need(t, name, q.device)
        if t.dtype == torch.float8_e4m3fn:
            t = t.view(torch.uint8)
        if t.dtype != torch.uint8:
            raise ValueError(f"{name} must be uint8 (e4m3 / e8m0 bytes)")
        return t
    q, k, v = raw(q, "q"), raw(k, "k"), raw(v, "v")
    qs, ks, vs = raw(q_scale, "q_scale"), raw(k_scale, "k_scale"), raw(v_scale, "v_scale")
    if q.dim() != 4 or k.dim() != 4 or k.shape != v.shape:
        raise ValueError("q must be [B, Hq, S, 128] and k, v [B, Hkv, S, 128]")
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    if k.shape[0] != B or k.shape[2] != S or k.shape[3] != D:
        raise ValueError("k and v must be [batch, kv_heads, seq, head_dim]")
    if (qs.shape != (B, Hq, S, D // 32) or ks.shape != (B, Hkv, S, D // 32)
            or vs.shape != (B, Hkv, -(-S // 32), D)):
        raise ValueError("scales must be [B, Hq, S, D/32], [B, Hkv, S, D/32] and "
                         "[B, Hkv, ceil(S/32), D]")
    odt = _dtype(out_dtype)
    out = _out(out, (B, Hq, S, D), odt, q.device)
    if lse is not None:
        _need(lse, "lse", q.device)
        if lse.dtype != torch.float32 or lse.shape != (B, Hq, S):
            raise ValueError("lse must be float32 [B, Hq, S]")
    rt.check(rt.lib().wave_fa_fwd_mxfp8_launch(
        q.data_ptr(), qs.data_ptr(), k.data_ptr(), ks.data_ptr(), v.data_ptr(), vs.data_ptr(),
        out.data_ptr(), lse.data_ptr() if lse is not None else None, B, Hq, Hkv, S, D,
        _DT[odt], int(causal), float(scale or 0.0), _stream(q)))
    return out


def flash_attention_lse(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                        causal: bool = False, scale: float | None = None
                        ) -> tuple[torch.Tensor, torch.Tensor]:
    """The online-softmax forward plus each row's log-sum-exp
    lse[b, h, q] = ln sum_k exp(scale * q.k) (float32), for flash_attention_bwd
    (wave_fa_fwd_lse_launch)."""
    B, Hq, Hkv, S, D = _fa_shapes(q, k, v)
    out = torch.empty_like(q)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device=q.device)
    rt.check(rt.lib().wave_fa_fwd_lse_launch(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(), B, Hq, Hkv, S,
        D, _DT[q.dtype], int(causal), float(scale or 0.0), _stream(q)))
    return out, lse


def flash_attention_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                        do: torch.Tensor, lse: torch.Tensor, *, causal: bool = False,
                        scale: float | None = None
                        ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """dQ, dK, dV of O = softmax(scale Q K^T) V given dO, O and the forward's
    lse (flash_attention_lse); wave_fa_bwd_launch.  seq % 64 == 0."""
    B, Hq, Hkv, S, D = _fa_shapes(q, k, v)
    for t, n in ((o, "o"), (do, "do")):
        _need(t, n, q.device)
        if t.shape != q.shape or t.dtype != q.dtype:
            raise ValueError(f"{n} must match q")
    _need(lse, "lse", q.device)
    if lse.dtype != torch.float32 or tuple(lse.shape) != (B, Hq, S):
        raise ValueError("lse must be float32 [batch, q_heads, seq]")
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    delta = torch.empty((B, Hq, S), dtype=torch.float32, device=q.device)
    rt.check(rt.lib().wave_fa_bwd_launch(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(), lse.data_ptr(),
        delta.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, Hq, Hkv, S, D,
        _DT[q.dtype], int(causal), float(scale or 0.0), _stream(q)))
    return dq, dk, dv


def flash_attention_f32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        out: torch.Tensor | None = None) -> torch.Tensor:
    """The flash_attention_f32 ABI: q [block_m, D] f16 pre-scaled by
    log2(e)/sqrt(D), k/v [seq_n, D] f16 -> O [block_m, D] f32 (exp2 softmax)."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _need(t, n, q.device)
        if t.dim() != 2 or t.dtype != torch.float16:
            raise ValueError(f"{n} must be a 2-D f16 tensor")
    block_m, D = q.shape
    seq_n = k.shape[0]
    if k.shape[1] != D or v.shape != k.shape:
        raise ValueError("k and v must both be [seq_n, head_dim] with q's head_dim")
    out = _out(out, (block_m, D), torch.float32, q.device)
    rt.check(rt.lib().wave_fa_f32_launch(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), block_m, seq_n, D,
        _stream(q)))
    return out
