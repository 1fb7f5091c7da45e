"""RWKV-7 WKV recurrence on MI355X: the reference's Python surface over the HIP library (include/wkv7.h).

Per head the state S (K x V, fp32) evolves as

    S_t = diag(d_t) S_{t-1} + b_t (a_t^T S_{t-1}) + k_t v_t^T          d_t = exp(-exp(w_t))
    o_t = S_t^T r_t

(rwkv_next/kernels/wkv7.py:4-7).  Same names, argument meanings and return values as the reference module
rwkv_next/kernels/wkv7.py:
    wkv7(r, w, k, v, a, b, state, H, K, cu_seqlens=None, final=True) -> (o, ht | None)      (wkv7.py:126-138)
    wkv7_replay(r, w, k, v, a, b, state, n_keep, H, K) -> state   (in place)                (wkv7.py:141-147)
    torch op rwkv_next::wkv7_fwd (also rwkv_next_amd::wkv7_fwd), functional, for torch.compile (wkv7.py:113-123)
plus the slot-pool entry the reference builds around the op in the model (model.py:366-371, 382-396, 485):
    wkv7_pool_(r, w, k, v, a, b, pool, slots, H, K, ...) -> o     (pool updated in place, optional snapshots)
The in-place entries are registered torch ops too (rwkv_next_amd::wkv7_pool_, rwkv_next_amd::wkv7_replay_, with
their mutated arguments declared and fake implementations), so a torch.compile'd caller such as the reference's
part_att (model.py:334-342) traces through them without a graph break.

Layouts: r, w, k, v, a, b (B, T, H*K) bf16 (w RAW); states (N, H, K, K) fp32; o like v.  Head size K: 64 (every
RWKV-7 model) runs the specialised kernels; any other 1 <= K <= 256 (the reference pads K to a power of two and masks,
wkv7.py:55-59, 96) runs a generic token-serial kernel with the same features, and algo AUTO or RECURRENT.
All work runs in HIP kernels on the current stream; nothing here synchronises, so every entry point can be
captured in a CUDA/HIP graph.  There is no CPU or PyTorch fallback.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from .. import _lib
from ._workspace import stream_workspace

_WORKSPACES: dict = {}  # (device index, stream handle) -> [workspace, flags zeroed in stream order, capture id]


def reset_workspaces() -> None:
    """Drop the cached per-stream workspaces (the next call creates a zeroed one)."""
    _WORKSPACES.clear()

HEAD_SIZE = 64      # every RWKV-7 model's head size: the specialised kernels
MAX_HEAD_SIZE = 256  # other head sizes run the generic token-serial kernel
OPERANDS = ("r", "w", "k", "v", "a", "b")


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _prep_operands(r, w, k, v, a, b, H, K):
    if not 1 <= K <= MAX_HEAD_SIZE:
        raise ValueError(f"head size K={K} is not supported (1 <= K <= {MAX_HEAD_SIZE})")
    ops = [r, w, k, v, a, b]
    shape = r.shape
    for name, t in zip(OPERANDS, ops):
        if t.shape != shape:
            raise ValueError(f"operand {name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
        if t.dtype != torch.bfloat16:
            raise TypeError(f"operand {name} must be bfloat16 (got {t.dtype})")
        if t.device.type != "cuda":
            raise ValueError(f"operand {name} must be on a GPU (got {t.device})")
    if r.dim() == 4:
        B, T = shape[0], shape[1]
        if shape[2] != H or shape[3] != K:
            raise ValueError(f"operands (B, T, H, K) = {tuple(shape)} do not match H={H}, K={K}")
    elif r.dim() == 3:
        B, T = shape[0], shape[1]
        if shape[2] != H * K:
            raise ValueError(f"operands (B, T, H*K) = {tuple(shape)} do not match H={H}, K={K}")
    else:
        raise ValueError(f"operands must be (B, T, H*K) or (B, T, H, K), got {tuple(shape)}")
    ops = [t.contiguous() for t in ops]  # the reference does the same (wkv7.py:129, 144)
    return ops, B, T


def _state_arg(state, rows_expected, H, K, name="state"):
    if state is None:
        return None
    if state.dtype != torch.float32:
        raise TypeError(f"{name} must be float32 (got {state.dtype})")
    if tuple(state.shape[1:]) != (H, K, K):
        raise ValueError(f"{name} must be (N, {H}, {K}, {K}), got {tuple(state.shape)}")
    if rows_expected is not None and state.shape[0] != rows_expected:
        raise ValueError(f"{name} has {state.shape[0]} rows, expected {rows_expected}")
    return state.contiguous()


def _launch(ops, *, H, K=HEAD_SIZE, num_seqs, T, total, o=None, h0=None, h0_idx=None, h0_rows=0, ht=None,
            ht_idx=None, ht_rows=0, fresh=None, cu=None, n_keep=None, snap=None, algo=_lib.ALGO_AUTO, rec_max_len=-1,
            status=None):
    dev = ops[0].device
    args = _lib.Wkv7Args()
    for name, t in zip(OPERANDS, ops):
        setattr(args, name, t.data_ptr())
    args.in_tok_stride = H * K
    args.o = _ptr(o)
    args.o_tok_stride = H * K
    args.h0, args.h0_idx, args.h0_rows = _ptr(h0), _ptr(h0_idx), h0_rows
    args.ht, args.ht_idx, args.ht_rows = _ptr(ht), _ptr(ht_idx), ht_rows
    args.fresh = _ptr(fresh)
    args.cu_seqlens = _ptr(cu)
    args.n_keep = _ptr(n_keep)
    args.snapshots = _ptr(snap)
    args.num_seqs, args.T, args.total_tokens = num_seqs, T, total
    args.H, args.head_size, args.algo, args.rec_max_len = H, K, algo, rec_max_len
    args.status = _ptr(status)
    nbytes = _lib.workspace_size(args)
    ws = None
    if nbytes:
        # one workspace per (device, stream): its leading flag region starts zero and every call leaves it zero
        ws = stream_workspace(_WORKSPACES, dev, nbytes, _lib.WKV7_FLAG_REGION_BYTES)
        args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    with torch.cuda.device(dev):
        _lib.run(args, torch.cuda.current_stream(dev).cuda_stream)
    return ws


def _index_tensor(x, dev, dtype, name):
    if x is None:
        return None
    x = torch.as_tensor(x, device=dev)
    if x.dtype != dtype:
        x = x.to(dtype)
    return x.contiguous()


# --------------------------------------------------------------------------------------------------------------
# functional forward (reference: _wkv7_op / wkv7)
# --------------------------------------------------------------------------------------------------------------
def _fwd_impl(r, w, k, v, a, b, h0, H: int, K: int, final: bool, algo: int = _lib.ALGO_AUTO):
    ops, B, T = _prep_operands(r, w, k, v, a, b, H, K)
    h0 = _state_arg(h0 if (h0 is not None and h0.numel()) else None, B, H, K, "h0")
    o = torch.empty_like(ops[3])
    ht = torch.empty(B, H, K, K, device=r.device, dtype=torch.float32) if final else r.new_empty(0,
                                                                                              dtype=torch.float32)
    _launch(ops, H=H, K=K, num_seqs=B, T=T, total=B * T, o=o, h0=h0, h0_rows=B, ht=ht if final else None, ht_rows=B,
            algo=algo)
    return o, ht


def _wkv7_fwd(r: Tensor, w: Tensor, k: Tensor, v: Tensor, a: Tensor, b: Tensor, h0: Tensor, H: int, K: int,
              final: bool) -> tuple[Tensor, Tensor]:
    """Functional form (fresh o and final state) with the schema of the reference's rwkv_next::wkv7_fwd
    (rwkv_next/kernels/wkv7.py:113-123).  h0 may be empty (0 rows) for a zero initial state."""
    return _fwd_impl(r, w, k, v, a, b, h0, H, K, final)


def _wkv7_fwd_fake(r, w, k, v, a, b, h0, H, K, final):
    B = r.shape[0]
    o = v.new_empty(v.shape)  # contiguous, like the real output (empty_like would keep a strided v's strides)
    return o, (r.new_empty(B, H, K, K, dtype=torch.float32) if final else r.new_empty(0, dtype=torch.float32))


wkv7_fwd = torch.library.custom_op("rwkv_next_amd::wkv7_fwd", _wkv7_fwd, mutates_args=())
wkv7_fwd.register_fake(_wkv7_fwd_fake)


def _op_registered(namespace: str, name: str) -> bool:
    """Whether torch.ops.<namespace>.<name> exists in this process (any registration: custom_op, triton_op, a
    schema from torch.library.define)."""
    try:
        getattr(getattr(torch.ops, namespace), name)
    except (AttributeError, RuntimeError):
        return False
    return True


def _register_reference_name():
    """The same op under the reference's name, rwkv_next::wkv7_fwd, so that callers binding torch.ops.rwkv_next
    find it.  Skipped (returns None) when that name is already registered in this process, e.g. by the reference
    package itself: registering again would silently replace that op (torch accepts a second registration of a
    name and dispatches to the later one)."""
    if _op_registered("rwkv_next", "wkv7_fwd"):
        return None
    op = torch.library.custom_op("rwkv_next::wkv7_fwd", _wkv7_fwd, mutates_args=())
    op.register_fake(_wkv7_fwd_fake)
    return op


wkv7_fwd_reference_name = _register_reference_name()


def wkv7(r, w, k, v, a, b, state, H, K, cu_seqlens=None, final=True, *, algo: int = _lib.ALGO_AUTO):
    """o, final_state = recurrence over (B, T, H*K) inputs from `state` (B|N, H, K, K) fp32 or None.
    w is RAW (decay = exp(-exp(w))).  cu_seqlens (N+1,) int32: packed varlen (B must be 1).
    Rows longer than 32 tokens run the chunked form, which needs w <= 1.0 (RWKV-7's w = -softplus(-x) - 0.5 is
    always below -0.5); larger w needs algo=ALGO_RECURRENT (the status word of wkv7_pool_ reports it).
    Mirrors rwkv_next/kernels/wkv7.py:126-138."""
    if cu_seqlens is None:
        if algo == _lib.ALGO_AUTO:
            h0 = state.contiguous() if state is not None else r.new_empty(0, dtype=torch.float32)
            o, ht = wkv7_fwd(r, w, k, v, a, b, h0, H, K, final)
        else:
            o, ht = _fwd_impl(r, w, k, v, a, b, state, H, K, final, algo)
        return o, (ht if final else None)
    ops, B, T = _prep_operands(r, w, k, v, a, b, H, K)
    if B != 1:
        raise ValueError("cu_seqlens requires B == 1 (packed varlen)")
    cu = _index_tensor(cu_seqlens, r.device, torch.int32, "cu_seqlens")
    N = cu.numel() - 1
    h0 = _state_arg(state, N, H, K, "state")
    o = torch.empty_like(ops[3])
    ht = torch.empty(N, H, K, K, device=r.device, dtype=torch.float32) if final else None
    _launch(ops, H=H, K=K, num_seqs=N, T=0, total=T, o=o, h0=h0, h0_rows=N, ht=ht, ht_rows=N, cu=cu, algo=algo)
    return o, ht


def _require(t: Tensor, name: str, dtype, shape) -> None:
    """Raise ValueError unless `t` is a contiguous tensor of `dtype` and `shape` (None entries match any size).
    The registered ops hand raw pointers to the C ABI, so a strided or mis-shaped buffer would be read and written
    at the wrong elements instead of failing."""
    if t.dtype != dtype or not t.is_contiguous() or t.dim() != len(shape) or \
            any(want is not None and got != want for got, want in zip(t.shape, shape)):
        want = ", ".join("*" if x is None else str(x) for x in shape)
        raise ValueError(f"{name} must be a contiguous {dtype} ({want}) tensor, got {t.dtype} {tuple(t.shape)} "
                         f"{'contiguous' if t.is_contiguous() else 'strided'}")


@torch.library.custom_op("rwkv_next_amd::wkv7_replay_", mutates_args=("state",))
def wkv7_replay_(r: Tensor, w: Tensor, k: Tensor, v: Tensor, a: Tensor, b: Tensor, state: Tensor, n_keep: Tensor,
                 H: int, K: int) -> None:
    """In-place rollback as a registered op: state (B, H, K, K) fp32 := the recurrence over the first n_keep[b]
    steps of row b.  The body of the reference's wkv7_replay (rwkv_next/kernels/wkv7.py:141-147)."""
    ops, B, T = _prep_operands(r, w, k, v, a, b, H, K)
    _require(state, "state", torch.float32, (B, H, K, K))
    _require(n_keep, "n_keep", torch.int64, (B,))
    _launch(ops, H=H, K=K, num_seqs=B, T=T, total=B * T, h0=state, h0_rows=B, ht=state, ht_rows=B, n_keep=n_keep,
            algo=_lib.ALGO_RECURRENT)


@wkv7_replay_.register_fake
def _(r, w, k, v, a, b, state, n_keep, H, K):
    return None


def wkv7_replay(r, w, k, v, a, b, state, n_keep, H, K):
    """Rollback: state (B, H, K, K) fp32 := the recurrence over the first n_keep[b] steps of row b, IN PLACE.
    No output is computed.  Mirrors rwkv_next/kernels/wkv7.py:141-147."""
    B = r.shape[0]
    if state.dtype != torch.float32 or not state.is_contiguous() or tuple(state.shape) != (B, H, K, K):
        raise ValueError(f"state must be a contiguous float32 ({B}, {H}, {K}, {K}) tensor")
    nk = _index_tensor(n_keep, r.device, torch.int64, "n_keep")
    if nk.numel() != B:
        raise ValueError(f"n_keep has {nk.numel()} entries, expected {B}")
    wkv7_replay_(r, w, k, v, a, b, state, nk, H, K)
    return state


# --------------------------------------------------------------------------------------------------------------
# slot-pool entry (the model's decode / prefill / verify call sites, model.py:366-371, 382-396, 485)
# --------------------------------------------------------------------------------------------------------------
@torch.library.custom_op("rwkv_next_amd::wkv7_pool_", mutates_args=("pool", "snapshots", "status"))
def wkv7_pool_op(r: Tensor, w: Tensor, k: Tensor, v: Tensor, a: Tensor, b: Tensor, pool: Tensor, slots: Tensor,
                 H: int, K: int, cu_seqlens: Optional[Tensor], n_keep: Optional[Tensor], fresh: Optional[Tensor],
                 final: bool, store_o: bool, snapshots: Optional[Tensor], status: Optional[Tensor], max_len: int,
                 algo: int, rec_max_len: int) -> Tensor:
    """The slot-pool recurrence as a registered op (arguments already checked and converted by wkv7_pool_).
    Returns o, or an empty tensor when store_o is False."""
    ops, B, T = _prep_operands(r, w, k, v, a, b, H, K)
    if cu_seqlens is not None:
        _require(cu_seqlens, "cu_seqlens", torch.int32, (None,))
        N, Tn, total = cu_seqlens.numel() - 1, max_len, T
    else:
        N, Tn, total = B, T, B * T
    _require(pool, "pool", torch.float32, (None, H, K, K))
    _require(slots, "slots", torch.int64, (N,))
    if n_keep is not None:
        _require(n_keep, "n_keep", torch.int64, (N,))
    if fresh is not None:
        _require(fresh, "fresh", torch.uint8, (N,))
    if snapshots is not None:
        _require(snapshots, "snapshots", torch.float32, (N, Tn, H, K, K))
    if status is not None:
        _require(status, "status", torch.int32, (None,))
        if status.numel() < 1:
            raise ValueError("status must hold at least one int32")
    o = torch.empty_like(ops[3]) if store_o else ops[3].new_empty(0)
    _launch(ops, H=H, K=K, num_seqs=N, T=Tn, total=total, o=o if store_o else None, h0=pool, h0_idx=slots,
            h0_rows=pool.shape[0], ht=pool if final else None, ht_idx=slots if final else None,
            ht_rows=pool.shape[0], fresh=fresh, cu=cu_seqlens, n_keep=n_keep, snap=snapshots, algo=algo,
            rec_max_len=rec_max_len, status=status)
    return o


@wkv7_pool_op.register_fake
def _(r, w, k, v, a, b, pool, slots, H, K, cu_seqlens, n_keep, fresh, final, store_o, snapshots, status, max_len,
      algo, rec_max_len):
    return v.new_empty(v.shape) if store_o else v.new_empty(0)


def wkv7_pool_(r, w, k, v, a, b, pool, slots, H, K, *, cu_seqlens=None, n_keep=None, fresh=None, final=True,
               store_o=True, snapshots=None, max_len: int = 0, algo: int = _lib.ALGO_AUTO,
               rec_max_len: int = -1, check_slots: bool = False, status=None):
    """Recurrence for N sequences whose states live in `pool` (S, H, K, K) fp32, updated IN PLACE.

    slots (N,) int64: pool row of each sequence (must be distinct).  Dense operands (N, T, H*K), or packed
    (1, sumT, H*K) with cu_seqlens (N+1,) int32.  fresh (N,) bool: start those rows from zeros (the reference
    zeroes them first, model.py:382-383).  n_keep (N,) int64: run only the first n_keep[n] tokens.
    final=False reads the pool without writing it (speculative verify, model.py:475-496).
    snapshots: optional (N, T, H, K, K) fp32 receiving the state after every token (ragged calls: (N, max_len, H,
    K, K), row n's entries t < its length written, the rest untouched); rolling back to an accepted prefix of n
    tokens is `restore_snapshots_(pool, slots, snapshots, n)`.  Snapshot calls run the token-serial kernel.
    max_len: ragged calls may pass an upper bound on any row's length (sizes the workspace and the snapshot rows;
    0 = sumT); a longer row is cut to its first max_len tokens and reported through status (WKV7_STATUS_SEQLENS).
    status: optional int32 device tensor (one element, see new_status): a check launched ahead of the recurrence
    ORs WKV7_STATUS_* bits into it when a slot index lies outside the pool, cu_seqlens is malformed or an n_keep
    entry is negative (the kernels skip such reads and writes and go on), when a call that runs the chunked
    kernels has w above 1.0 (their results are not finite: the chunked form needs w <= 1.0, which RWKV-7's
    w = -softplus(-x) - 0.5 always meets), or, for calls of at most 1024 rows, when two rows share a slot (their
    states race).  Nothing synchronises: read it with check_status when convenient.
    Returns o like v (or None when store_o=False).  Runs as the registered op rwkv_next_amd::wkv7_pool_."""
    if r.dim() not in (3, 4):
        raise ValueError(f"operands must be (B, T, H*K) or (B, T, H, K), got {tuple(r.shape)}")
    B, T = r.shape[0], r.shape[1]
    dev = r.device
    if pool.dtype != torch.float32 or not pool.is_contiguous() or tuple(pool.shape[1:]) != (H, K, K):
        raise ValueError(f"pool must be a contiguous float32 (S, {H}, {K}, {K}) tensor")
    sl = _index_tensor(slots, dev, torch.int64, "slots")
    if cu_seqlens is not None:
        if B != 1:
            raise ValueError("cu_seqlens requires B == 1 (packed varlen)")
        cu = _index_tensor(cu_seqlens, dev, torch.int32, "cu_seqlens")
        N = cu.numel() - 1
    else:
        cu, N = None, B
    if sl.numel() != N:
        raise ValueError(f"slots has {sl.numel()} entries, expected {N}")
    if check_slots:  # host sync: for tests and debugging, not for the graphed hot path
        check_distinct_slots(sl, pool.shape[0])
    nk = _index_tensor(n_keep, dev, torch.int64, "n_keep")
    fr = None
    if fresh is not None:
        fr = torch.as_tensor(fresh, device=dev)
        fr = (fr if fr.dtype == torch.uint8 else fr.to(torch.uint8)).contiguous()
    if snapshots is not None:
        if cu is not None and max_len < 1:
            raise ValueError("ragged calls with snapshots need max_len >= 1 (the snapshot rows' length)")
        Ts = T if cu is None else int(max_len)
        if snapshots.dtype != torch.float32 or not snapshots.is_contiguous() or \
                tuple(snapshots.shape) != (N, Ts, H, K, K):
            raise ValueError(f"snapshots must be a contiguous float32 ({N}, {Ts}, {H}, {K}, {K}) tensor")
    if status is not None and (status.dtype != torch.int32 or status.numel() < 1 or status.device != dev):
        raise ValueError("status must be an int32 tensor of at least one element on the operands' device")
    o = wkv7_pool_op(r, w, k, v, a, b, pool, sl, H, K, cu, nk, fr, final, store_o, snapshots, status,
                     int(max_len), int(algo), int(rec_max_len))
    return o if store_o else None


def new_status(device) -> torch.Tensor:
    """A zeroed status word for wkv7_pool_(..., status=...)."""
    return torch.zeros(1, dtype=torch.int32, device=device)


STATUS_REASONS = {_lib.WKV7_STATUS_H0_SLOT: "initial-state slot index outside the pool",
                  _lib.WKV7_STATUS_HT_SLOT: "final-state slot index outside the pool",
                  _lib.WKV7_STATUS_SEQLENS: "cu_seqlens not non-decreasing within [0, total tokens]",
                  _lib.WKV7_STATUS_NKEEP: "negative n_keep",
                  _lib.WKV7_STATUS_DECAY: f"w above {_lib.WKV7_CHUNK_W_MAX} on a call that runs the chunked kernels "
                                          "(their results are not finite): run it with algo=ALGO_RECURRENT",
                  _lib.WKV7_STATUS_SLOT_CLASH: "two sequences share a state slot (a final state stored where another "
                                               "sequence stores or reads its state): the result depends on timing",
                  _lib.WKV7_STATUS_SEGMENT_WAIT: "the segmented prefill gave up waiting for a segment hand-off: "
                                                 "the results are wrong and the stream's workspace flags must be "
                                                 "zeroed (reset_workspaces())"}


def check_status(status: torch.Tensor) -> None:
    """Raise ValueError naming every WKV7_STATUS_* bit set in `status` (synchronises the host: call it outside
    graph capture and the hot loop)."""
    bits = int(status.reshape(-1)[0].item())
    if bits:
        raise ValueError("wkv7: " + "; ".join(m for bit, m in STATUS_REASONS.items() if bits & bit))


def check_distinct_slots(slots: torch.Tensor, num_slots: int) -> None:
    """Raise if slot indices repeat or fall outside [0, num_slots).  Duplicate slots in one in-place call race
    (the reference's index_copy_ is nondeterministic for them, model.py:396).  Synchronises the host."""
    s = slots.detach().to("cpu")
    if s.numel() and (int(s.min()) < 0 or int(s.max()) >= num_slots):
        raise ValueError(f"slot index outside [0, {num_slots})")
    if torch.unique(s).numel() != s.numel():
        raise ValueError("duplicate slot indices in one call")


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def restore_snapshots_(pool, slots, snapshots, n):
    """Rollback after a speculative verify: pool[slots[b]] := snapshots[b, n[b] - 1], the state after the first
    n[b] tokens (1 <= n[b] <= T); rows with n[b] = 0 keep the pool's state (a verify with final=False does not
    write the pool).  Replaces the reference's second recurrence pass, wkv7_replay (model.py:498-508), with one
    HIP copy kernel (16 KB read + 16 KB written per (row, head)); no host sync.  slots must be distinct."""
    if pool.dtype != torch.float32 or not pool.is_contiguous() or pool.dim() != 4 or pool.shape[2:] != (64, 64):
        raise ValueError("pool must be a contiguous float32 (S, H, 64, 64) tensor")
    N, T, H = snapshots.shape[0], snapshots.shape[1], pool.shape[1]
    if snapshots.dtype != torch.float32 or not snapshots.is_contiguous() or \
            tuple(snapshots.shape) != (N, T, H, 64, 64):
        raise ValueError(f"snapshots must be a contiguous float32 (N, T, {H}, 64, 64) tensor")
    dev = pool.device
    sl = _index_tensor(slots, dev, torch.int64, "slots")
    nn = _index_tensor(n, dev, torch.int64, "n")
    if sl.numel() != N or nn.numel() != N:
        raise ValueError(f"slots and n must have {N} entries")
    with torch.cuda.device(dev):
        _lib.check(_lib.load().wkv7_snapshot_restore(pool.data_ptr(), pool.shape[0], H, sl.data_ptr(),
                                                     snapshots.data_ptr(), T, nn.data_ptr(), N, _stream(dev)))
    return pool


# --------------------------------------------------------------------------------------------------------------
# model-level wrapper and the per-model state pool (model.py:77-83, 298-316)
# --------------------------------------------------------------------------------------------------------------
def model_wkv7(r, w, k, v, a, b, state, H, N, cu_seqlens=None, final=True):
    """RWKV-7 recurrence for (B, T, H*N) inputs of any float dtype (cast to bf16); `w` is the raw log-decay.
    Returns (o (B, T, C) bf16, new_state fp32 | None).  Mirrors the model's wrapper, rwkv_next/model.py:77-83."""
    B, T, C = r.shape
    bf = lambda t: t if t.dtype == torch.bfloat16 else t.bfloat16()
    o, s = wkv7(bf(r), bf(w), bf(k), bf(v), bf(a), bf(b), state, H, N, cu_seqlens, final)
    return o.view(B, T, C), s


class StatePool:
    """fp32 WKV state for `layers` layers x `slots` slots x H heads, (L, S, H, 64, 64) -- the WKV part of the
    reference model's slot pool (alloc_slots / state_bytes_per_slot / reset_slots / move_slots,
    rwkv_next/model.py:298-316).  Layer i's pool `pool.layer(i)` (S, H, 64, 64) is what `wkv7_pool_` updates in
    place; reset and move run as HIP kernels on the current stream (graph-capturable, no host sync)."""

    def __init__(self, layers: int, slots: int, H: int, device, N: int = HEAD_SIZE):
        if N != HEAD_SIZE:  # the slot reset / move / restore kernels are built for the model's 64 x 64 states
            raise ValueError(f"head size {N} is not supported by the state pool (N = {HEAD_SIZE})")
        self.L, self.S, self.H = int(layers), int(slots), int(H)
        self.device = torch.device(device)
        self.wkv = torch.zeros(self.L, self.S, self.H, N, N, device=self.device, dtype=torch.float32)

    def layer(self, i: int) -> torch.Tensor:
        return self.wkv[i]

    def state_bytes_per_slot(self) -> int:
        """WKV bytes per slot over all layers (the reference adds the two token-shift rows, model.py:307-308)."""
        return self.L * self.H * HEAD_SIZE * HEAD_SIZE * 4

    def reset_slots(self, idx) -> None:
        """wkv[:, idx] = 0 (model.py:310-311)."""
        i = _index_tensor(idx, self.device, torch.int64, "idx")
        with torch.cuda.device(self.device):
            _lib.check(_lib.load().wkv7_pool_reset(self.wkv.data_ptr(), self.L, self.S, self.H, i.data_ptr(),
                                                   i.numel(), _stream(self.device)))

    # ---- speculative decoding (the WKV part of rwkv_next/model.py:475-508) -----------------------------------
    def snapshot_buffer(self, B: int, T: int) -> torch.Tensor:
        """Per-layer state snapshots for a verify of T tokens on B rows: (L, B, T, H, 64, 64) fp32 (the
        reference keeps the operands instead and replays them)."""
        return torch.empty(self.L, int(B), int(T), self.H, HEAD_SIZE, HEAD_SIZE, device=self.device,
                           dtype=torch.float32)

    def verify_(self, i: int, r, w, k, v, a, b, slots, snapshots: torch.Tensor):
        """Layer i of a speculative verify (model.py:475-496, the wkv call with final=False): reads the states of
        `slots`, writes nothing to the pool, and records the state after every token in snapshots[i].  Returns o."""
        return wkv7_pool_(r, w, k, v, a, b, self.wkv[i], slots, self.H, HEAD_SIZE, final=False,
                          snapshots=snapshots[i])

    def rollback_(self, slots, n, snapshots: torch.Tensor) -> None:
        """wkv[:, slots[b]] := the state after the first n[b] verified tokens (1 <= n[b] <= T; 0 keeps the slot),
        layer by layer -- the WKV part of model.rollback (model.py:498-503), which replays the first n[b] recorded
        steps with wkv7_replay; here one copy kernel per layer restores snapshots[i][b, n[b] - 1].  No host sync,
        graph-capturable."""
        if snapshots.dim() != 6 or snapshots.shape[0] != self.L:
            raise ValueError(f"snapshots must be ({self.L}, B, T, {self.H}, 64, 64)")
        for i in range(self.L):
            restore_snapshots_(self.wkv[i], slots, snapshots[i], n)

    def replay_(self, i: int, r, w, k, v, a, b, slots, n) -> None:
        """The reference's rollback for layer i (model.py:498-503, wkv7_replay): wkv[i, slots[b]] := the recurrence
        over the first n[b] of the verified tokens, in place (n[b] = 0 keeps the slot).  Bit-identical to rollback_ after a verify_ with
        snapshots (one fixed per-token instruction sequence); cheaper per speculative step when the snapshots are not
        needed otherwise (measured at B = 64, T = 5, H = 64: verify without snapshots + replay 58 us, verify with
        snapshots + restore 98 us)."""
        wkv7_pool_(r, w, k, v, a, b, self.wkv[i], slots, self.H, HEAD_SIZE, n_keep=n, store_o=False)

    def move_slots(self, src, dst) -> None:
        """wkv[:, dst] = wkv[:, src] with gather-then-scatter semantics (swaps are exact); dst must be distinct
        (model.py:313-316)."""
        s = _index_tensor(src, self.device, torch.int64, "src")
        d = _index_tensor(dst, self.device, torch.int64, "dst")
        if s.numel() != d.numel():
            raise ValueError("src and dst must have the same length")
        if s.numel() > _lib.MAX_MOVES:
            raise ValueError(f"at most {_lib.MAX_MOVES} moves per call")
        with torch.cuda.device(self.device):
            _lib.check(_lib.load().wkv7_pool_move(self.wkv.data_ptr(), self.L, self.S, self.H, s.data_ptr(),
                                                  d.data_ptr(), s.numel(), _stream(self.device)))
