"""Tensor-level operators over the gfx950 kernel library.

Each operator validates dtype, device, contiguity and shape, allocates any
output the caller did not pass, and launches the HIP kernel on the current
torch stream through the C-ABI (``_lib``).  Launches are asynchronous, like
the reference harnesses' ``ct.launch`` (e.g. cutile-attn-gqa/main.py:249-252):
the caller synchronises.  There is no CPU path: inputs must be on a HIP
device and the native library must be present.
"""
from __future__ import annotations

import math

import torch

from . import _lib

_IO_DTYPES = {torch.bfloat16: _lib.MX_DTYPE_BF16, torch.float16: _lib.MX_DTYPE_F16}


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _require(t: torch.Tensor, name: str, dtypes, ndim: int | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype not in dtypes:
        raise TypeError(f"{name} has dtype {t.dtype}, expected one of {list(dtypes)}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a HIP device (got {t.device})")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must be {ndim}-D (got shape {tuple(t.shape)})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _same_device(*ts: torch.Tensor) -> None:
    devs = {t.device for t in ts}
    if len(devs) != 1:
        raise ValueError(f"all tensors must be on one device (got {sorted(map(str, devs))})")


def gemm_bf16(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """C = A @ B for row-major bf16 A[M,K], B[K,N]; fp32 accumulate, bf16 C.

    Semantics of cutile-matmul-tc-bf16/main.py:59-78.
    """
    _require(a, "a", (torch.bfloat16,), 2)
    _require(b, "b", (torch.bfloat16,), 2)
    M, K = a.shape
    K2, N = b.shape
    if K != K2:
        raise ValueError(f"inner dimensions differ: a {tuple(a.shape)} vs b {tuple(b.shape)}")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    _require(out, "out", (torch.bfloat16,), 2)
    if tuple(out.shape) != (M, N):
        raise ValueError(f"out must be {(M, N)}, got {tuple(out.shape)}")
    _same_device(a, b, out)
    _lib.call("mx_gemm_bf16", a.data_ptr(), b.data_ptr(), out.data_ptr(), M, N, K, K, N, N, _stream())
    return out


def gemm_fp8_bs(a: torch.Tensor, sa: torch.Tensor, b: torch.Tensor, sb: torch.Tensor,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """Block-scaled e4m3 GEMM, bf16 out.

    a[M,K], b[K,N]: torch.float8_e4m3fn; sa[M, K/128], sb[K/128, ceil(N/128)]:
    fp32 dequantisation scales.  C[m,n] = sum_kb sa[m,kb] sb[kb,n//128] *
    (A[m,kb-block] . B[kb-block,n]).
    """
    f8 = (torch.float8_e4m3fn,)
    _require(a, "a", f8, 2)
    _require(b, "b", f8, 2)
    _require(sa, "sa", (torch.float32,), 2)
    _require(sb, "sb", (torch.float32,), 2)
    M, K = a.shape
    K2, N = b.shape
    if K != K2:
        raise ValueError(f"inner dimensions differ: a {tuple(a.shape)} vs b {tuple(b.shape)}")
    if K % 128:
        raise ValueError(f"K={K} must be a multiple of 128 (scale block depth)")
    if tuple(sa.shape) != (M, K // 128):
        raise ValueError(f"sa must be {(M, K // 128)}, got {tuple(sa.shape)}")
    if tuple(sb.shape) != (K // 128, (N + 127) // 128):
        raise ValueError(f"sb must be {(K // 128, (N + 127) // 128)}, got {tuple(sb.shape)}")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    _require(out, "out", (torch.bfloat16,), 2)
    if tuple(out.shape) != (M, N):
        raise ValueError(f"out must be {(M, N)}, got {tuple(out.shape)}")
    _same_device(a, sa, b, sb, out)
    _lib.call("mx_gemm_fp8_bs", a.data_ptr(), sa.data_ptr(), b.data_ptr(), sb.data_ptr(), out.data_ptr(),
              M, N, K, _stream())
    return out


def gqa_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
            scale: float | None = None, out: torch.Tensor | None = None, block_m: int | None = None,
            block_n: int | None = None, wave_m: int | None = None) -> torch.Tensor:
    """Fused GQA forward.  q [B,Hq,S,D]; k, v [B,Hkv,S,D]; bf16 or f16.

    Semantics of cutile-attn-gqa/main.py:64-170 (scale defaults to 1/sqrt(D)
    as in :85) with an optional causal mask.  block_m / block_n / wave_m
    select the tile (mx_gqa_fwd_tile: query rows of a head per workgroup,
    keys per LDS stage, query rows per wave); unset ones take the default
    tile's value, and a tile the library has no kernel for raises MXError.
    """
    _require(q, "q", _IO_DTYPES, 4)
    _require(k, "k", (q.dtype,), 4)
    _require(v, "v", (q.dtype,), 4)
    B, Hq, S, D = q.shape
    Bk, Hkv, Sk, Dk = k.shape
    if (Bk, Sk, Dk) != (B, S, D) or tuple(v.shape) != tuple(k.shape):
        raise ValueError(f"shape mismatch: q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    if Hq % Hkv:
        raise ValueError(f"n_q ({Hq}) must be divisible by n_kv ({Hkv})")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty_like(q)
    _require(out, "out", (q.dtype,), 4)
    if out.shape != q.shape:
        raise ValueError(f"out must be {tuple(q.shape)}")
    _same_device(q, k, v, out)
    if block_m is None and block_n is None and wave_m is None:
        _lib.call("mx_gqa_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, Hq, Hkv, S, D,
                  float(scale), int(bool(causal)), _IO_DTYPES[q.dtype], _stream())
        return out
    bm = gqa_default_block_m(Hq, Hkv, D) if block_m is None else int(block_m)
    bn = 64 if block_n is None else int(block_n)
    wm = 32 if wave_m is None else int(wave_m)
    _lib.call("mx_gqa_fwd_tile", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, Hq, Hkv, S, D,
              float(scale), int(bool(causal)), _IO_DTYPES[q.dtype], bm, bn, wm, _stream())
    return out


def gqa_default_block_m(n_q: int, n_kv: int, d_head: int) -> int:
    """BLOCK_M of the default GQA tile (queries of a head per workgroup)."""
    r = int(_lib.load().mx_gqa_fwd_default_block_m(n_q, n_kv, d_head))
    if r < 0:
        raise ValueError(f"no GQA tile for n_q={n_q} n_kv={n_kv} d={d_head}: {_lib.strerror(r)}")
    return r


def gqa_tile_supported(n_q: int, n_kv: int, d_head: int, block_m: int, block_n: int = 64, wave_m: int = 32) -> bool:
    """Whether mx_gqa_fwd_tile has a kernel for this tile (host logic, no GPU call)."""
    return int(_lib.load().mx_gqa_fwd_tile_check(n_q, n_kv, d_head, block_m, block_n, wave_m)) == 0


def gqa_tile_info(n_q: int, n_kv: int, d_head: int, dtype: torch.dtype, causal: bool, block_m: int,
                  block_n: int = 64, wave_m: int = 32) -> tuple[int, int]:
    """(registers per lane, scratch bytes per lane) of the kernel a tile runs."""
    import ctypes

    regs, scratch = ctypes.c_int(0), ctypes.c_int(0)
    _lib.call("mx_gqa_fwd_tile_info", n_q, n_kv, d_head, _IO_DTYPES[dtype], int(bool(causal)), block_m, block_n,
              wave_m, ctypes.byref(regs), ctypes.byref(scratch))
    return regs.value, scratch.value


def mla_decode_workspace_bytes(B: int, H: int, T: int, d_latent: int = 512) -> int:
    return int(_lib.load().mx_mla_decode_workspace(B, H, T, d_latent))


def mla_decode_splits(B: int, H: int, T: int) -> int:
    """How many slices of T the decode splits each sequence into (1: no merge)."""
    return int(_lib.load().mx_mla_decode_splits(B, H, T))


def mla_prefill_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
                    scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Pre-projected MLA prefill attention, every head its own K/V.

    Semantics of cutile-attn-mla/main.py:81-163 (scale defaults to
    1/sqrt(qk_head_dim)) without its zero padding of qk_head_dim to a power
    of two: q, k [B,H,S,d_qk], v [B,H,S,d_v] -> out [B,H,S,d_v], bf16 or
    f16.  (d_qk, d_v) in {(192,128), (96,64), (128,128), (64,64)}.
    """
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _require(t, n, _IO_DTYPES, 4)
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, v must share a dtype")
    B, H, S, Dqk = q.shape
    if tuple(k.shape) != (B, H, S, Dqk) or tuple(v.shape[:3]) != (B, H, S):
        raise ValueError(f"shape mismatch: q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    Dv = v.shape[3]
    if scale is None:
        scale = 1.0 / math.sqrt(Dqk)
    if out is None:
        out = torch.empty((B, H, S, Dv), dtype=q.dtype, device=q.device)
    _require(out, "out", (q.dtype,), 4)
    if tuple(out.shape) != (B, H, S, Dv):
        raise ValueError(f"out must be {(B, H, S, Dv)}")
    _same_device(q, k, v, out)
    _lib.call("mx_mla_prefill_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), B, H, S, Dqk, Dv,
              float(scale), int(bool(causal)), _IO_DTYPES[q.dtype], _stream())
    return out


def mla_decode(q: torch.Tensor, kv: torch.Tensor, scale: float, d_latent: int = 512,
               out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Absorbed MLA decode.  q [B,H,576], kv [B,T,576] bf16 -> out [B,H,512].

    out[b,h] = softmax(scale * q[b,h] . kv[b]^T) . kv[b][:, :d_latent].
    """
    _require(q, "q", (torch.bfloat16,), 3)
    _require(kv, "kv", (torch.bfloat16,), 3)
    B, H, Dq = q.shape
    Bk, T, Dk = kv.shape
    if Bk != B or Dk != Dq:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)} kv {tuple(kv.shape)}")
    d_rope = Dq - d_latent
    if out is None:
        out = torch.empty((B, H, d_latent), dtype=torch.bfloat16, device=q.device)
    _require(out, "out", (torch.bfloat16,), 3)
    if tuple(out.shape) != (B, H, d_latent):
        raise ValueError(f"out must be {(B, H, d_latent)}")
    need = mla_decode_workspace_bytes(B, H, T, d_latent)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_ptr = workspace.data_ptr() if (need and workspace is not None) else None
    ws_bytes = workspace.numel() * workspace.element_size() if (need and workspace is not None) else 0
    _same_device(q, kv, out)
    _lib.call("mx_mla_decode", q.data_ptr(), kv.data_ptr(), out.data_ptr(), B, H, T, d_latent, d_rope,
              float(scale), ws_ptr, ws_bytes, _stream())
    return out


def gdn_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, alpha: torch.Tensor, beta: torch.Tensor,
               S_in: torch.Tensor, S_out: torch.Tensor | None = None,
               o: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Gated-DeltaNet decode step.  Returns (o, S_out).

    q, k [B,Hk,dk]; v [B,Hv,dv] (bf16 or f16); alpha, beta [B,Hv] fp32;
    S_in [B,Hv,dk,dv] fp32.  S_out may be S_in for an in-place update.
    Semantics of cutile-attn-gdn/main.py:92-185 with Hk != Hv grouping.
    """
    _require(q, "q", _IO_DTYPES, 3)
    _require(k, "k", (q.dtype,), 3)
    _require(v, "v", (q.dtype,), 3)
    _require(alpha, "alpha", (torch.float32,), 2)
    _require(beta, "beta", (torch.float32,), 2)
    _require(S_in, "S_in", (torch.float32,), 4)
    B, Hk, dk = q.shape
    Bv, Hv, dv = v.shape
    if tuple(k.shape) != (B, Hk, dk) or Bv != B:
        raise ValueError(f"shape mismatch: q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    if Hv % Hk:
        raise ValueError(f"n_v_heads ({Hv}) must be a multiple of n_k_heads ({Hk})")
    if tuple(alpha.shape) != (B, Hv) or tuple(beta.shape) != (B, Hv):
        raise ValueError(f"alpha/beta must be {(B, Hv)}")
    if tuple(S_in.shape) != (B, Hv, dk, dv):
        raise ValueError(f"S_in must be {(B, Hv, dk, dv)}, got {tuple(S_in.shape)}")
    if S_out is None:
        S_out = torch.empty_like(S_in)
    _require(S_out, "S_out", (torch.float32,), 4)
    if S_out.shape != S_in.shape:
        raise ValueError("S_out must match S_in")
    if o is None:
        o = torch.empty((B, Hv, dv), dtype=q.dtype, device=q.device)
    _require(o, "o", (q.dtype,), 3)
    if tuple(o.shape) != (B, Hv, dv):
        raise ValueError(f"o must be {(B, Hv, dv)}")
    _same_device(q, k, v, alpha, beta, S_in, S_out, o)
    _lib.call("mx_gdn_decode", q.data_ptr(), k.data_ptr(), v.data_ptr(), alpha.data_ptr(), beta.data_ptr(),
              S_in.data_ptr(), S_out.data_ptr(), o.data_ptr(), B, Hk, Hv, dk, dv, _IO_DTYPES[q.dtype],
              _stream())
    return o, S_out


def gdn_block_v(B: int, Hv: int, dk: int, dv: int) -> int:
    """Width of the d_v column blocks the GDN/KDA kernels use for this
    problem (the reference's `pick_block_v`, cutile-attn-gdn/main.py:228-246)."""
    bv = int(_lib.load().mx_gdn_decode_block_v(B, Hv, dk, dv))
    if bv <= 0:
        raise ValueError(f"unsupported GDN/KDA sizes B={B} Hv={Hv} dk={dk} dv={dv}")
    return bv


def kda_decode(q, k, v, g, beta, S_in, S_out=None, o=None):
    """One KDA decode step (cutile-attn-kda/main.py:187-271): GDN with the
    per-channel decay exp(g) on the rows of the state.  q, k, g [B,H,dk];
    v [B,H,dv]; beta [B,H] (all bf16 or f16); S_in [B,H,dk,dv] fp32.
    Returns (o [B,H,dv], S_out).  S_out may be S_in (in-place update)."""
    _require(q, "q", _IO_DTYPES, 3)
    for t, n in ((k, "k"), (v, "v"), (g, "g")):
        _require(t, n, (q.dtype,), 3)
    _require(beta, "beta", (q.dtype,), 2)
    _require(S_in, "S_in", (torch.float32,), 4)
    B, Hh, dk = q.shape
    dv = v.shape[2]
    if tuple(k.shape) != (B, Hh, dk) or tuple(g.shape) != (B, Hh, dk) or tuple(v.shape[:2]) != (B, Hh):
        raise ValueError(f"shape mismatch: q {tuple(q.shape)} k {tuple(k.shape)} g {tuple(g.shape)} v {tuple(v.shape)}")
    if tuple(beta.shape) != (B, Hh):
        raise ValueError(f"beta must be {(B, Hh)}")
    if tuple(S_in.shape) != (B, Hh, dk, dv):
        raise ValueError(f"S_in must be {(B, Hh, dk, dv)}, got {tuple(S_in.shape)}")
    if S_out is None:
        S_out = torch.empty_like(S_in)
    _require(S_out, "S_out", (torch.float32,), 4)
    if S_out.shape != S_in.shape:
        raise ValueError("S_out must match S_in")
    if o is None:
        o = torch.empty((B, Hh, dv), dtype=q.dtype, device=q.device)
    _require(o, "o", (q.dtype,), 3)
    if tuple(o.shape) != (B, Hh, dv):
        raise ValueError(f"o must be {(B, Hh, dv)}")
    _same_device(q, k, v, g, beta, S_in, S_out, o)
    _lib.call("mx_kda_decode", q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
              S_in.data_ptr(), S_out.data_ptr(), o.data_ptr(), B, Hh, dk, dv, _IO_DTYPES[q.dtype], _stream())
    return o, S_out


def quant_fp8_act(x, q=None, scales=None):
    """fp8 activation quantisation with 1x128 block scales (the producer of
    gemm_fp8_bs's A operand): x [M,K] bf16/f16 (K % 128 == 0) ->
    (q [M,K] float8_e4m3fn, scales [M,K/128] fp32) with x ~= q * scale."""
    _require(x, "x", _IO_DTYPES, 2)
    M, K = x.shape
    if K % 128:
        raise ValueError(f"K ({K}) must be a multiple of 128")
    if q is None:
        q = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=x.device)
    _require(q, "q", (torch.float8_e4m3fn,), 2)
    if scales is None:
        scales = torch.empty((M, K // 128), dtype=torch.float32, device=x.device)
    _require(scales, "scales", (torch.float32,), 2)
    if tuple(q.shape) != (M, K) or tuple(scales.shape) != (M, K // 128):
        raise ValueError(f"q must be {(M, K)} and scales {(M, K // 128)}")
    _same_device(x, q, scales)
    _lib.call("mx_quant_fp8_act", x.data_ptr(), q.data_ptr(), scales.data_ptr(), M, K, K, _IO_DTYPES[x.dtype],
              _stream())
    return q, scales


def gemm_bf16_batched(a, b, out=None):
    """C[i] = A[i] @ B[i] for contiguous bf16 A [batch,M,K], B [batch,K,N]."""
    _require(a, "a", (torch.bfloat16,), 3)
    _require(b, "b", (torch.bfloat16,), 3)
    nb, M, K = a.shape
    if b.shape[0] != nb or b.shape[1] != K:
        raise ValueError(f"shape mismatch: a {tuple(a.shape)} vs b {tuple(b.shape)}")
    N = b.shape[2]
    if out is None:
        out = torch.empty((nb, M, N), dtype=torch.bfloat16, device=a.device)
    _require(out, "out", (torch.bfloat16,), 3)
    if tuple(out.shape) != (nb, M, N):
        raise ValueError(f"out must be {(nb, M, N)}")
    _same_device(a, b, out)
    _lib.call("mx_gemm_bf16_batched", a.data_ptr(), b.data_ptr(), out.data_ptr(), nb, M, N, K, K, N, N,
              M * K, K * N, M * N, _stream())
    return out


def _head_gemm(x, w, out, out_ld):
    """out[:, h, :] = x[:, h, :] @ w[h] for every head, x [B,H,K] and w
    [H,K,N] contiguous; out rows are out_ld elements apart per head slot."""
    B, Hh, K = x.shape
    N = w.shape[2]
    _lib.call("mx_gemm_bf16_batched", x.data_ptr(), w.data_ptr(), out.data_ptr(), Hh, B, N, K, Hh * K, N,
              Hh * out_ld, K, K * N, out_ld, _stream())


def mla_absorb_q(q_nope, w_uk, out=None):
    """Weight absorption of the MLA query: q_lat[b,h,:] = q_nope[b,h,:] @ W_UK[h]
    (MECHANISMS.md:91-94: q^T (W_UK c) = (W_UK^T q)^T c).  q_nope [B,H,dn],
    w_uk [H,dn,d_c] bf16 -> q_lat [B,H,d_c] bf16 (fp32 accumulate)."""
    _require(q_nope, "q_nope", (torch.bfloat16,), 3)
    _require(w_uk, "w_uk", (torch.bfloat16,), 3)
    B, Hh, dn = q_nope.shape
    if w_uk.shape[0] != Hh or w_uk.shape[1] != dn:
        raise ValueError(f"w_uk must be [{Hh}, {dn}, d_c], got {tuple(w_uk.shape)}")
    dc = w_uk.shape[2]
    if out is None:
        out = torch.empty((B, Hh, dc), dtype=torch.bfloat16, device=q_nope.device)
    _require(out, "out", (torch.bfloat16,), 3)
    if tuple(out.shape) != (B, Hh, dc):
        raise ValueError(f"out must be {(B, Hh, dc)}")
    _same_device(q_nope, w_uk, out)
    _head_gemm(q_nope, w_uk, out, dc)
    return out


def mla_up_project(o_lat, w_uv, out=None):
    """Output up-projection of the absorbed MLA decode: o[b,h,:] =
    o_lat[b,h,:] @ W_UV[h] (MECHANISMS.md:115-120).  o_lat [B,H,d_c],
    w_uv [H,d_c,dv] bf16 -> o [B,H,dv] bf16."""
    _require(o_lat, "o_lat", (torch.bfloat16,), 3)
    _require(w_uv, "w_uv", (torch.bfloat16,), 3)
    B, Hh, dc = o_lat.shape
    if w_uv.shape[0] != Hh or w_uv.shape[1] != dc:
        raise ValueError(f"w_uv must be [{Hh}, {dc}, dv], got {tuple(w_uv.shape)}")
    dv = w_uv.shape[2]
    if out is None:
        out = torch.empty((B, Hh, dv), dtype=torch.bfloat16, device=o_lat.device)
    _require(out, "out", (torch.bfloat16,), 3)
    if tuple(out.shape) != (B, Hh, dv):
        raise ValueError(f"out must be {(B, Hh, dv)}")
    _same_device(o_lat, w_uv, out)
    _head_gemm(o_lat, w_uv, out, dv)
    return out


def mla_decode_absorbed_workspace_bytes(B: int, H: int, T: int) -> int:
    return int(_lib.load().mx_mla_decode_absorbed_workspace(B, H, T))


def mla_decode_absorbed(q_nope, q_rope, kv, w_uk, w_uv, scale, out=None, workspace=None):
    """Full weight-absorbed MLA decode step (MECHANISMS.md:77-94, 115-120):
    q_lat = q_nope @ W_UK[h], latent attention of [q_lat, q_rope] over the
    KV cache, o = o_lat @ W_UV[h] — one C-ABI call (mx_mla_decode_absorbed).
    q_nope [B,H,dn], q_rope [B,H,64], kv [B,T,576], w_uk [H,dn,512],
    w_uv [H,512,dv], all bf16 -> o [B,H,dv].  Pass `workspace` (uint8, at
    least mla_decode_absorbed_workspace_bytes) to allocate nothing."""
    for t, n in ((q_nope, "q_nope"), (q_rope, "q_rope"), (kv, "kv"), (w_uk, "w_uk"), (w_uv, "w_uv")):
        _require(t, n, (torch.bfloat16,), 3)
    B, Hh, dn = q_nope.shape
    T = kv.shape[1]
    if tuple(q_rope.shape) != (B, Hh, 64) or kv.shape[0] != B or kv.shape[2] != 576:
        raise ValueError(f"q_rope must be {(B, Hh, 64)} and kv [B, T, 576]")
    if tuple(w_uk.shape) != (Hh, dn, 512) or w_uv.shape[0] != Hh or w_uv.shape[1] != 512:
        raise ValueError(f"w_uk must be {(Hh, dn, 512)} and w_uv [{Hh}, 512, dv]")
    dv = w_uv.shape[2]
    if out is None:
        out = torch.empty((B, Hh, dv), dtype=torch.bfloat16, device=q_nope.device)
    _require(out, "out", (torch.bfloat16,), 3)
    if tuple(out.shape) != (B, Hh, dv):
        raise ValueError(f"out must be {(B, Hh, dv)}")
    need = mla_decode_absorbed_workspace_bytes(B, Hh, T)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need + 256, dtype=torch.uint8, device=q_nope.device)
    ws_ptr = (workspace.data_ptr() + 255) // 256 * 256
    ws_bytes = workspace.numel() * workspace.element_size() - (ws_ptr - workspace.data_ptr())
    _same_device(q_nope, q_rope, kv, w_uk, w_uv, out, workspace)
    _lib.call("mx_mla_decode_absorbed", q_nope.data_ptr(), q_rope.data_ptr(), kv.data_ptr(), w_uk.data_ptr(),
              w_uv.data_ptr(), out.data_ptr(), B, Hh, T, dn, dv, float(scale), ws_ptr, ws_bytes, _stream())
    return out
