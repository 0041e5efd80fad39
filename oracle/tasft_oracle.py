"""CPU oracle of the TASFT block-sparse attention path — TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference semantics, used as the checker of the HIP kernels.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import it; the product package ``tasft_amd`` never does.

Every function cites the reference lines it restates. Inputs are float arrays (the
bf16-rounded device inputs upcast to float32); arithmetic is float32 unless ``dtype``
asks for float64. How each function is pinned (checked independently of itself):

* ``pool_to_blocks``: literal vectors of tests/unit/test_numerical_correctness.py:40-98.
* ``gate_logits_concat``: textbook composition, checked against torch.nn.Linear/ReLU.
* ``gate_logits``: equals ``gate_logits_concat`` (the decomposition W.[x;y] = Wq x + Wk y).
* ``threshold_mask``: sigmoid via torch.sigmoid; invariants of
  tests/unit/test_causal_gate_and_single_pass.py:154-270 and test_edge_cases.py:207-238.
* ``attention_dense_masked``: torch SDPA for all-true masks (causal and not), and a
  pure-Python loop implementation on tiny inputs.
* ``attention_block_gather``: equals ``attention_dense_masked``.
* ``sparse_decode``: equals the last row of ``attention_block_gather``; brute force.
* ``sparse_decode_paged``: equals ``sparse_decode`` on the contiguous cache from which the
  test scatters the page pools through a random page permutation.
* ``attention_varlen``: equals ``attention_dense_masked`` over the whole packed token
  range with an independently built block-diagonal token mask (tests/test_oracle.py), and
  with one sequence equals the reference's flat-token call (B = 1).
* ``gate_target_from_scores``: literal vectors of tests/unit/test_objectives.py:169-191,
  test_numerical_correctness.py:119-157 and :714-721; torch max_pool2d + softmax.
* ``block_max`` / ``gate_target_from_qk``: equal ``gate_target_from_scores`` applied to
  explicitly built scores.
* ``gate_kl_loss``: torch ``F.kl_div(..., reduction="batchmean")`` composed as the reference
  does (tests/test_oracle.py); ``gate_kl_grad``: torch autograd of that composition.
* ``sparsity_stats`` / ``estimate_speedup``: literal values of tests/unit/test_kernel.py.
* ``mask_to_csr`` / ``indices_to_mask``: a hand-checked literal example and the round
  trip dense -> CSR -> dense (numpy ``nonzero`` / fancy-index scatter).
"""
from __future__ import annotations

import math

import numpy as np


# ----------------------------------------------------------------------------- gate
def pool_to_blocks(x: np.ndarray, bs: int) -> np.ndarray:
    """Zero-padded block mean ``[..., S, D] -> [..., NB, D]`` (attn_gate.py:151-175).

    The mean divides by ``bs`` even for the padded last block (pad zeros count).
    """
    s = x.shape[-2]
    pad = (bs - s % bs) % bs
    if pad:
        widths = [(0, 0)] * x.ndim
        widths[-2] = (0, pad)
        x = np.pad(x, widths)
    nb = x.shape[-2] // bs
    return x.reshape(*x.shape[:-2], nb, bs, x.shape[-1]).mean(axis=-2)


def gate_logits_concat(qbar: np.ndarray, kbar: np.ndarray, w_in: np.ndarray, b_in: np.ndarray,
                       w_out: np.ndarray) -> np.ndarray:
    """Logits from the materialised pair concat (attn_gate.py:248-257).

    ``qbar [..., NBq, D]``, ``kbar [..., NBk, D]`` (same leading dims), ``w_in [hid, 2D]``,
    ``b_in [hid]``, ``w_out [1, hid]`` -> ``[..., NBq, NBk]``. Cat order is (q, k) (:253).
    """
    nbq, d = qbar.shape[-2:]
    nbk = kbar.shape[-2]
    lead = qbar.shape[:-2]
    q_exp = np.broadcast_to(qbar[..., :, None, :], (*lead, nbq, nbk, d))
    k_exp = np.broadcast_to(kbar[..., None, :, :], (*lead, nbq, nbk, d))
    cat = np.concatenate([q_exp, k_exp], axis=-1)
    hidden = np.maximum(cat @ w_in.T + b_in, 0.0)
    return (hidden @ w_out.reshape(-1, 1))[..., 0]


def gate_logits(q: np.ndarray, k: np.ndarray, w_in: np.ndarray, b_in: np.ndarray, w_out: np.ndarray,
                bs: int, dtype: type = np.float32) -> np.ndarray:
    """Gate logits ``[B, Hq, NB, NB]`` for ``q [B,Hq,S,D]``, ``k [B,Hkv,S,D]``.

    Uses ``W_in.[x; y] = W_in[:, :D] x + W_in[:, D:] y`` (exact algebra of attn_gate.py:253-256)
    so the per-pair cost is ``hid`` instead of ``2D x hid``; K head ``h // G`` serves query
    head ``h`` (the repeat_interleave of tasft_attention.py:725-729).
    """
    d = q.shape[-1]
    g = q.shape[1] // k.shape[1]
    qb = pool_to_blocks(q.astype(dtype), bs)
    kb = np.repeat(pool_to_blocks(k.astype(dtype), bs), g, axis=1)
    w = w_in.astype(dtype)
    uq = qb @ w[:, :d].T + b_in.astype(dtype)
    uk = kb @ w[:, d:].T
    wo = w_out.astype(dtype).reshape(-1)
    out = np.empty(qb.shape[:3] + (kb.shape[2],), dtype=dtype)
    for b in range(q.shape[0]):
        for h in range(q.shape[1]):
            hid = np.maximum(uq[b, h][:, None, :] + uk[b, h][None, :, :], 0.0)
            out[b, h] = hid @ wo
    return out


def sigmoid(x: np.ndarray) -> np.ndarray:
    return 1.0 / (1.0 + np.exp(-x))


def threshold_mask(logits: np.ndarray, tau, causal: bool) -> tuple[np.ndarray, np.ndarray]:
    """Soft scores and hard mask from logits (attn_gate.py:259-275).

    ``tau`` is a float or per-head array ``[H]``. With ``causal`` the upper block triangle
    of the soft scores is exactly 0, and the mask there is ``0 >= tau``.
    """
    soft = sigmoid(logits.astype(np.float32)).astype(np.float32)
    if causal:
        nb = soft.shape[-1]
        soft = soft * np.tril(np.ones((nb, nb), dtype=np.float32))
    t = np.asarray(tau, dtype=np.float32)
    if t.ndim == 1:
        t = t.reshape(1, -1, 1, 1)
    return soft, soft >= t


# ----------------------------------------------------------------------------- attention
def token_mask(block_mask: np.ndarray, s: int, bs: int, causal: bool) -> np.ndarray:
    """Element mask of the reference kernel (block_sparse_fa.py:192-243, host prep :502-508)."""
    m = block_mask.astype(bool)
    nb = m.shape[-1]
    if causal:
        m = m & np.tril(np.ones((nb, nb), dtype=bool))
    tm = np.repeat(np.repeat(m, bs, axis=-2), bs, axis=-1)[..., :s, :s]
    if causal:
        tm = tm & np.tril(np.ones((s, s), dtype=bool))
    return tm


def attention_dense_masked(q, k, v, block_mask, bs: int, causal: bool = True,
                           scale: float | None = None, dtype: type = np.float32) -> np.ndarray:
    """``softmax(QK^T*scale + M) V`` with M from ``token_mask``; empty rows give 0.

    Restates the kernel's math (block_sparse_fa.py:228-258): scale after the dot
    product (:228), -inf outside the mask (:243), and the division by
    ``where(l > 0, l, 1)`` (:255-257), so an empty row gives 0 and a row whose sum is NaN
    (a NaN score among its keys) stays NaN.
    GQA: query head h uses K/V head h // G. No bf16 rounding of P (the kernel's P->bf16
    cast at :252 is inside the tolerance).
    """
    b_, hq, s, d = q.shape
    g = hq // k.shape[1]
    sc = scale if scale is not None else 1.0 / math.sqrt(d)
    out = np.zeros(q.shape, dtype=dtype)
    for b in range(b_):
        for h in range(hq):
            tm = token_mask(block_mask[b, h], s, bs, causal)
            sco = (q[b, h].astype(dtype) @ k[b, h // g].astype(dtype).T) * dtype(sc)
            sco = np.where(tm, sco, -np.inf)
            mx = sco.max(axis=-1, keepdims=True)
            has = np.isfinite(mx)
            p = np.exp(sco - np.where(has, mx, 0.0))
            l = p.sum(axis=-1, keepdims=True)
            o = p @ v[b, h // g].astype(dtype)
            out[b, h] = o / np.where(l > 0, l, 1.0)
    return out


def attention_block_gather(q, k, v, block_mask, bs: int, causal: bool = True,
                           scale: float | None = None, dtype: type = np.float32,
                           heads: list[tuple[int, int]] | None = None) -> np.ndarray:
    """Same result as ``attention_dense_masked``, computing only the active blocks.

    For each query block, the active key blocks (block_sparse_fa.py:192-203) are gathered
    and one softmax is taken over their tokens. ``heads`` restricts the work to the given
    (b, h) pairs (other rows stay 0) — used for bounded CPU timing samples.
    """
    b_, hq, s, d = q.shape
    g = hq // k.shape[1]
    nb = math.ceil(s / bs)
    sc = dtype(scale if scale is not None else 1.0 / math.sqrt(d))
    out = np.zeros(q.shape, dtype=dtype)
    pairs = heads if heads is not None else [(b, h) for b in range(b_) for h in range(hq)]
    for b, h in pairs:
        qh = q[b, h].astype(dtype)
        kh = k[b, h // g].astype(dtype)
        vh = v[b, h // g].astype(dtype)
        for i in range(nb):
            q0, q1 = i * bs, min((i + 1) * bs, s)
            kbs = [j for j in range(nb) if block_mask[b, h, i, j] and (not causal or j <= i)]
            if not kbs:
                continue
            idx = np.concatenate([np.arange(j * bs, min((j + 1) * bs, s)) for j in kbs])
            sco = (qh[q0:q1] @ kh[idx].T) * sc
            if causal:
                sco = np.where(idx[None, :] <= np.arange(q0, q1)[:, None], sco, -np.inf)
            mx = sco.max(axis=-1, keepdims=True)
            p = np.exp(sco - np.where(np.isfinite(mx), mx, 0.0))
            l = p.sum(axis=-1, keepdims=True)
            out[b, h, q0:q1] = (p @ vh[idx]) / np.where(l > 0, l, 1.0)
    return out


def attention_varlen(q, k, v, cu_seqlens, block_mask, bs: int, causal: bool = True,
                     scale: float | None = None, dtype: type = np.float32) -> np.ndarray:
    """Packed variable-length prefill: ``attention_block_gather`` per sequence.

    q ``[T, Hq, D]``, k/v ``[T, Hkv, D]`` (the flat token layout of
    tasft/inference/vllm_patch.py:172-176); sequence n is tokens ``cu_seqlens[n] ..
    cu_seqlens[n+1]-1`` and uses the leading corner of ``block_mask[n]`` (``[Hq, NB, NB]``).
    The reference views the whole packed range as one sequence (B = 1, :172-176); this
    keeps each request to its own tokens, with positions and blocks counted from its first
    token (the kernel semantics of block_sparse_fa.py:192-269 per sequence). Tokens after
    ``cu_seqlens[-1]`` stay 0.
    """
    cu = [int(x) for x in cu_seqlens]
    out = np.zeros(q.shape, dtype=dtype)
    for n in range(len(cu) - 1):
        t0, t1 = cu[n], cu[n + 1]
        if t1 <= t0:
            continue
        nb = math.ceil((t1 - t0) / bs)
        qs = q[t0:t1].transpose(1, 0, 2)[None]
        ks = k[t0:t1].transpose(1, 0, 2)[None]
        vs = v[t0:t1].transpose(1, 0, 2)[None]
        o = attention_block_gather(qs, ks, vs, block_mask[n:n + 1, :, :nb, :nb], bs, causal,
                                   scale, dtype)
        out[t0:t1] = o[0].transpose(1, 0, 2)
    return out


def sparse_decode(q, k_cache, v_cache, block_mask, bs: int, kv_lens=None,
                  scale: float | None = None, dtype: type = np.float32) -> np.ndarray:
    """Decode closed form: ``softmax(q K_sel^T*scale) V_sel`` over selected tokens < kv_len.

    ``q [B,Hq,1,D]``, caches ``[B,Hkv,S_kv,D]``, ``block_mask [B,Hq,1,NB]``. No reference
    function exists (decode is dense in tasft/inference/vllm_patch.py:189-196); this is the
    last query row of the prefill semantics (block_sparse_fa.py:192-258) with every cached
    token causally visible. A head with no selected token gives 0.
    """
    b_, hq, _, d = q.shape
    s_kv = k_cache.shape[2]
    g = hq // k_cache.shape[1]
    sc = dtype(scale if scale is not None else 1.0 / math.sqrt(d))
    out = np.zeros(q.shape, dtype=dtype)
    for b in range(b_):
        n = s_kv if kv_lens is None else int(min(max(kv_lens[b], 0), s_kv))
        for h in range(hq):
            sel = np.flatnonzero(block_mask[b, h, 0])
            idx = np.concatenate([np.arange(j * bs, min((j + 1) * bs, n)) for j in sel] or [np.zeros(0, int)])
            idx = idx[idx < n]
            if idx.size == 0:
                continue
            kh = k_cache[b, h // g, idx].astype(dtype)
            sco = (kh @ q[b, h, 0].astype(dtype)) * sc
            p = np.exp(sco - sco.max())
            out[b, h, 0] = (p @ v_cache[b, h // g, idx].astype(dtype)) / p.sum()
    return out


# ----------------------------------------------------------------------------- gate target
def sparse_decode_paged(q, k_pages, v_pages, block_table, kv_lens, block_mask, bs: int,
                        scale: float | None = None, dtype: type = np.float32) -> np.ndarray:
    """Sparse decode over a paged cache: gather each sequence's tokens, then ``sparse_decode``.

    Pools ``[pages, page_size, Hkv, D]`` in vLLM's block-table layout (the cache that
    tasft/inference/vllm_patch.py:189-196 hands to PagedAttention): token t of sequence b
    is row ``t % page_size`` of page ``block_table[b, t // page_size]``.
    """
    b_ = q.shape[0]
    ps, hkv, d = k_pages.shape[1], k_pages.shape[2], k_pages.shape[3]
    s_kv = block_mask.shape[-1] * bs
    k = np.zeros((b_, hkv, s_kv, d), dtype=k_pages.dtype)
    v = np.zeros((b_, hkv, s_kv, d), dtype=v_pages.dtype)
    for b in range(b_):
        for t in range(int(kv_lens[b])):
            page = int(block_table[b, t // ps])
            k[b, :, t] = k_pages[page, t % ps]
            v[b, :, t] = v_pages[page, t % ps]
    return sparse_decode(q, k, v, block_mask, bs, kv_lens, scale, dtype)


def _softmax(x: np.ndarray, axis: int) -> np.ndarray:
    mx = x.max(axis=axis, keepdims=True)
    e = np.exp(x - mx)
    return e / e.sum(axis=axis, keepdims=True)


def gate_target_from_scores(scores: np.ndarray, bs: int) -> np.ndarray:
    """-inf pad, block max-pool, softmax over the flat block grid (objectives.py:128-185).

    Raises ValueError on NaN or +inf (the reference raises NaNDetectedError, :148-164).
    """
    if np.isnan(scores).any() or np.isposinf(scores).any():
        raise ValueError("non-finite attention scores")
    b, h, sq, sk = scores.shape
    pq, pk = (bs - sq % bs) % bs, (bs - sk % bs) % bs
    x = np.pad(scores, ((0, 0), (0, 0), (0, pq), (0, pk)), constant_values=-np.inf)
    nbq, nbk = x.shape[2] // bs, x.shape[3] // bs
    pooled = x.reshape(b, h, nbq, bs, nbk, bs).max(axis=(3, 5))
    return _softmax(pooled.reshape(b, h, nbq * nbk), axis=-1).reshape(b, h, nbq, nbk)


def block_max(q, k, bs: int, causal: bool = True, scale: float | None = None,
              dtype: type = np.float32, attn_mask: np.ndarray | None = None) -> np.ndarray:
    """Raw pooled maxima of ``QK^T*scale (+ triu(-inf)) (+ attn_mask)``, ``[B,Hq,NB,NB]``.

    The scores are those of tasft_attention.py:426-449 (K head h // G for query head h):
    the causal ``triu(-inf, 1)`` term, then the additive ``attn_mask`` — ``[B, S]`` is
    broadcast as ``[:, None, None, :]`` (:446-448), a 4-D mask broadcasts to
    ``[B, Hq, S, S]``. Pooling as objectives.py:170-178. One query block at a time.
    """
    b_, hq, s, d = q.shape
    g = hq // k.shape[1]
    nb = math.ceil(s / bs)
    sc = dtype(scale if scale is not None else 1.0 / math.sqrt(d))
    out = np.full((b_, hq, nb, nb), -np.inf, dtype=dtype)
    pad = nb * bs - s
    am = None
    if attn_mask is not None:
        am = attn_mask[:, None, None, :] if attn_mask.ndim == 2 else attn_mask
        am = np.broadcast_to(am.astype(dtype), (b_, hq, s, s))
    for b in range(b_):
        for h in range(hq):
            kh = k[b, h // g].astype(dtype)
            for i in range(nb):
                q0, q1 = i * bs, min((i + 1) * bs, s)
                sco = (q[b, h, q0:q1].astype(dtype) @ kh.T) * sc
                if am is not None:
                    sco = sco + am[b, h, q0:q1]
                if causal:
                    sco = np.where(np.arange(s)[None, :] <= np.arange(q0, q1)[:, None], sco, -np.inf)
                if pad:
                    sco = np.pad(sco, ((0, 0), (0, pad)), constant_values=-np.inf)
                out[b, h, i] = sco.reshape(q1 - q0, nb, bs).max(axis=(0, 2))
    return out


def normalize_block_max(pooled: np.ndarray, normalize: str = "flat", temperature: float = 1.0,
                        clamp: float | None = None) -> np.ndarray:
    """Softmax of pooled maxima: flat grid (objectives.py:181-185) or per row.

    ``clamp``/``temperature`` follow tasft_attention.py:272-290: finite values are clamped
    to [-clamp, clamp], then divided by the temperature; -inf maps to 0.
    """
    x = pooled.astype(np.float64)
    if clamp is not None:
        x = np.where(np.isfinite(x), np.clip(x, -clamp, clamp), x)
    x = x / temperature
    b, h, nbq, nbk = x.shape
    if normalize == "flat":
        return _softmax(x.reshape(b, h, nbq * nbk), -1).reshape(b, h, nbq, nbk)
    if normalize == "row":
        return _softmax(x, -1)
    if normalize == "none":
        return x
    raise ValueError(normalize)


def gate_target_from_qk(q, k, bs: int, causal: bool = True, normalize: str = "flat",
                        temperature: float = 1.0, clamp: float | None = None,
                        scale: float | None = None, attn_mask: np.ndarray | None = None) -> np.ndarray:
    """``normalize_block_max(block_max(q, k))`` — the score producer plus compute_gate_target."""
    return normalize_block_max(block_max(q, k, bs, causal, scale, attn_mask=attn_mask), normalize,
                               temperature, clamp)


# ----------------------------------------------------------------------------- gate loss
KL_EPS = 1e-8  # objectives.py:39


def gate_kl_loss(soft: np.ndarray, target: np.ndarray) -> float:
    """KL(target || gate) with "batchmean" (objectives.py:187-221).

    Per (b, h) the scores are normalised over the flat NB_q*NB_k grid, ``g / (sum g + eps)``,
    then ``log(. + eps)``; entries with ``target == 0`` contribute 0; the sum over (b, h) is
    divided by B.
    """
    b, h = soft.shape[:2]
    g = soft.reshape(b, h, -1).astype(np.float64)
    t = target.reshape(b, h, -1).astype(np.float64)
    dist = g / (g.sum(-1, keepdims=True) + KL_EPS)
    logg = np.log(dist + KL_EPS)
    with np.errstate(divide="ignore", invalid="ignore"):
        terms = np.where(t > 0, t * (np.log(np.where(t > 0, t, 1.0)) - logg), 0.0)
    return float(terms.sum() / b)


def gate_kl_grad(soft: np.ndarray, target: np.ndarray) -> np.ndarray:
    """d gate_kl_loss / d soft: with Z = sum g + eps and u = g / Z + eps per (b, h),
    ``(-t_k / u_k + (sum_i t_i g_i / u_i) / Z) / (Z * B)``."""
    b, h = soft.shape[:2]
    g = soft.reshape(b, h, -1).astype(np.float64)
    t = target.reshape(b, h, -1).astype(np.float64)
    z = g.sum(-1, keepdims=True) + KL_EPS
    u = g / z + KL_EPS
    s2 = (t * g / u).sum(-1, keepdims=True)
    return ((-t / u + s2 / z) / (z * b)).reshape(soft.shape)


# ----------------------------------------------------------------------------- stats
def sparsity_stats(block_mask: np.ndarray) -> tuple[int, int, float]:
    """(total, active, sparsity) over the full grid (block_sparse_fa.py:586-588)."""
    total = int(block_mask.size)
    active = int(np.count_nonzero(block_mask))
    return total, active, 1.0 - active / max(total, 1)


def estimate_speedup(s: float) -> float:
    """``1 / max(1e-6, 1 - 0.98 s)`` (block_sparse_fa.py:616-618)."""
    return 1.0 / max(1e-6, 1.0 - s * 0.98)


# ----------------------------------------------------------------------------- formats
def mask_to_csr(mask: np.ndarray, causal: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """Dense block mask ``[B, H, NBq, NBk]`` -> CSR ``(row_ptr, col_idx)`` of the active blocks.

    Rows are ``(b, h, query block)`` row-major; columns ascend within a row. ``causal``
    keeps only key blocks <= the query block, the AND applied before the reference kernel
    (tasft/kernels/block_sparse_fa.py:502-508).
    """
    m = mask != 0
    if causal:
        nbq, nbk = m.shape[-2:]
        m = m & np.tril(np.ones((nbq, nbk), dtype=bool))
    rows = m.reshape(-1, m.shape[-1])
    counts = rows.sum(axis=1).astype(np.int64)
    row_ptr = np.zeros(rows.shape[0] + 1, dtype=np.int32)
    row_ptr[1:] = np.cumsum(counts)
    col_idx = np.nonzero(rows)[1].astype(np.int32)  # row-major order: ascending per row
    return row_ptr, col_idx


def indices_to_mask(indices: np.ndarray, num_blocks: int) -> np.ndarray:
    """Padded index lists ``[..., K]`` (``-1`` = empty) -> bool mask ``[..., num_blocks]``."""
    lead = indices.shape[:-1]
    flat = indices.reshape(-1, indices.shape[-1])
    out = np.zeros((flat.shape[0], num_blocks), dtype=bool)
    r, c = np.nonzero(flat >= 0)
    out[r, flat[r, c]] = True
    return out.reshape(*lead, num_blocks)
