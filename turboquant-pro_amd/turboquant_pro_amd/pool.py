"""GPU-resident two-tier TurboQuant KV cache for a batch of sequences.

``TQKVPool`` holds one attention layer's cache for up to ``max_batch``
sequences in HBM, in the layout documented in ``include/tqk.h``:

* coded groups live in pages (``page_tokens`` tokens x all kv heads) found
  through a per-sequence block table, with per-(group, head) metadata (NF4
  scale/mean, outlier side-list) in group slots found through a group table;
* the hot window is a per-(sequence, head) ring of ``hot_window`` tokens,
  fp16 (or fp32: ``input_dtype="float32"``, codes then from the fp32 values).

Appending runs the quantize-on-flush kernel for every group that the append
completes (the reference flush cadence: first flush at ``hot_window + 1``
tokens, then every ``(hot_window + 1) // 2``), then copies the surviving new
tokens into the ring.  Decoding runs the fused split-K kernel.  Host code only
plans launches; all per-token work is on the GPU.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np

from . import _native as N
from .formats import (NF4_ZERO_CODE, codes_from_key_rows, key_rows_from_codes, nf4_codes,
                      pack_key_codes, pack_values, tile_value_rows, uniform_codes, unpack_key_codes,
                      unpack_values, untile_value_rows)
from .codebooks import (HEAD_DIMS, dc_channel_mask, dc_mask_words, group_tokens_for, n_groups_for,
                        outliers_per_channel, random_rotation, rope_averaged_bias, value_codebook)

# key zero points; "symmetric" (symmetric NF4: no mean, per_channel_kv.py:354-357)
# is the descriptor's "sparse" mode with no DC channel, so every mean is 0
ZERO_POINTS = {"calibrated": 0, "sparse": 1, "bias": 2, "symmetric": 1}
# key forms: per-channel asym-NF4, per-channel uniform, PolarQuant (the value
# encode on the keys: per-token norms, rotated codes on the value codebook)
KEY_GRIDS = {"nf4_asym": 0, "uniform": 1, "polar": 2}


def _torch():
    import torch
    return torch


class TQKVPool:
    def __init__(self, n_kv_heads: int, n_q_heads: int | None = None, head_dim: int = 128, *,
                 max_batch: int = 1, max_seq_len: int = 8192, hot_window: int = 512,
                 key_bits: int = 4, value_bits: int = 3, outlier_frac: float = 0.02,
                 page_tokens: int | None = None, outlier_cap: int | None = None,
                 seed=None, rotation: tuple | None = None, block_table=None, device=None,
                 key_grid: str = "nf4_asym", zero_point: str = "calibrated",
                 rope_theta: float | None = None, k_bias=None, input_dtype: str = "float16"):
        torch = _torch()
        self._init_args = dict(n_kv_heads=n_kv_heads, n_q_heads=n_q_heads, head_dim=head_dim,
                               max_batch=max_batch, hot_window=hot_window, key_bits=key_bits,
                               value_bits=value_bits, outlier_frac=outlier_frac,
                               page_tokens=page_tokens, outlier_cap=outlier_cap, device=device,
                               key_grid=key_grid, zero_point=zero_point, rope_theta=rope_theta,
                               k_bias=k_bias, input_dtype=input_dtype)
        self._custom_table = block_table is not None
        if zero_point not in ZERO_POINTS:
            raise ValueError(f"zero_point must be one of {tuple(ZERO_POINTS)}")
        if key_grid not in KEY_GRIDS:
            raise ValueError(f"key_grid must be one of {tuple(KEY_GRIDS)}")
        if key_grid == "polar":
            if key_bits != value_bits:
                raise NotImplementedError("PolarQuant keys share the value codebook: key_bits must "
                                          "equal value_bits")
            outlier_frac = 0.0  # PolarQuant keys have no side-list
        if zero_point != "calibrated":
            if key_grid != "nf4_asym":
                raise ValueError(f"zero_point={zero_point!r} requires asym-NF4 keys")
            if rope_theta is None and zero_point != "symmetric":
                raise ValueError(f"zero_point={zero_point!r} requires rope_theta")
        if zero_point == "bias" and k_bias is None:
            raise ValueError('zero_point="bias" requires k_bias')
        if not torch.cuda.is_available():
            raise RuntimeError("TQKVPool runs on a ROCm GPU (gfx950); none is visible")
        self.device = torch.device(device if device is not None else "cuda")
        Hq = n_kv_heads if n_q_heads is None else n_q_heads
        G = group_tokens_for(hot_window)
        # default: 32-token pages (one decode block each) when groups are whole blocks
        P = (32 if G % 32 == 0 else G) if page_tokens is None else page_tokens
        k_out = outliers_per_channel(G, outlier_frac)
        if outlier_cap is None:
            outlier_cap = min(G * head_dim, 4 * k_out * head_dim) if k_out else 0
        max_groups = max(1, n_groups_for(max_seq_len, hot_window))
        max_pages = max(1, (max_groups * G + P - 1) // P) if P > 0 else 1
        if block_table is None and P == 32 and G % 32 == 0:
            # whole clusters of 8 groups per sequence (see _clustered_table)
            max_pages = -(-max_pages // (8 * (G // 32))) * (8 * (G // 32))
        self.n_kv_heads, self.n_q_heads, self.head_dim = n_kv_heads, Hq, head_dim
        self.max_batch, self.max_seq_len, self.hot_window = max_batch, max_seq_len, hot_window
        self.key_bits, self.value_bits, self.outlier_frac = key_bits, value_bits, outlier_frac
        self.group_tokens, self.page_tokens = G, P
        self.max_groups, self.max_pages = max_groups, max_pages
        if head_dim not in HEAD_DIMS:
            raise NotImplementedError(f"head_dim {head_dim}: the gfx950 kernels serve {HEAD_DIMS}")
        if input_dtype not in ("float16", "float32"):
            raise ValueError(f"input_dtype must be 'float16' or 'float32', not {input_dtype!r}")
        # fp32 caches: fp32 hot ring, query and appended tokens; codes from the
        # fp32 values (the VALU decode serves them)
        self.input_dtype = input_dtype
        self.f32 = input_dtype == "float32"
        # value codes in the MFMA-tiled byte order (see formats.py); head_dim
        # 128 and fp16 inputs only, the MFMA decode's
        self.tiled = head_dim == 128 and not self.f32 and (P % 16 == 0) and (G % 32 == 0)
        self.desc = N.CacheDesc(
            n_kv_heads=n_kv_heads, n_q_heads=Hq, head_dim=head_dim, hot_window=hot_window,
            group_tokens=G, page_tokens=P, key_bits=key_bits, value_bits=value_bits,
            outliers_per_channel=k_out, outlier_cap=outlier_cap,
            max_pages_per_seq=max_pages, max_groups_per_seq=max_groups,
            hot_ring=hot_window, n_pages=max_batch * max_pages, sm_scale=1.0 / math.sqrt(head_dim),
            key_grid=KEY_GRIDS[key_grid], zero_point=ZERO_POINTS[zero_point], input_f32=int(self.f32))
        self.key_grid = key_grid
        self.zero_point, self.rope_theta = zero_point, rope_theta
        # "sparse": the channels whose rotary wavelength exceeds a group
        self.dc_mask = (dc_channel_mask(rope_theta, head_dim, G) if zero_point == "sparse"
                        else np.zeros(head_dim, bool) if zero_point == "symmetric" else None)
        if self.dc_mask is not None:
            self.desc.dc_mask[:] = dc_mask_words(self.dc_mask)
        self.k_bias = None if k_bias is None else np.asarray(k_bias, np.float32).reshape(n_kv_heads, head_dim)
        N.check(N.lib().tqk_check_desc(ctypes.byref(self.desc)), "TQKVPool")

        dev = self.device
        n_pages = max_batch * max_pages
        n_slots = max_batch * max_groups
        u8, f32, i32, f16 = torch.uint8, torch.float32, torch.int32, torch.float16
        # head-major pages (include/tqk.h)
        self.kcodes = torch.zeros((n_kv_heads, n_pages, P, head_dim * key_bits // 8), dtype=u8, device=dev)
        self.vcodes = torch.zeros((n_kv_heads, n_pages, P, head_dim * value_bits // 8), dtype=u8, device=dev)
        self.vnorm = torch.zeros((n_kv_heads, n_pages, P), dtype=f32, device=dev)
        # PolarQuant keys: per-token key norms, laid out as vnorm
        self.knorm = (torch.zeros((n_kv_heads, n_pages, P), dtype=f32, device=dev)
                      if key_grid == "polar" else None)
        self.gscale = torch.zeros((n_slots, n_kv_heads, head_dim), dtype=f32, device=dev)
        self.gmean = torch.zeros((n_slots, n_kv_heads, head_dim), dtype=f32, device=dev)
        # cumulative outlier counts at every 32-token boundary of a group (last = total)
        self.ocount = torch.zeros((n_slots, n_kv_heads, 8), dtype=i32, device=dev)
        self.oent = torch.zeros((n_slots, n_kv_heads, max(outlier_cap, 1)), dtype=i32, device=dev)
        self.dtype = f32 if self.f32 else f16  # hot ring, appended tokens and queries
        self.hot_k = torch.zeros((max_batch, n_kv_heads, hot_window, head_dim), dtype=self.dtype, device=dev)
        self.hot_v = torch.zeros((max_batch, n_kv_heads, hot_window, head_dim), dtype=self.dtype, device=dev)
        if block_table is None:
            bt = self._clustered_table(max_batch, max_pages, P, G)
        else:
            bt = np.asarray(block_table, dtype=np.int32).reshape(max_batch, max_pages)
            if bt.min() < 0 or bt.max() >= n_pages:
                raise ValueError("block_table entries must index the page pool")
        self.block_table = torch.from_numpy(bt.copy()).to(dev)
        gt = np.arange(n_slots, dtype=np.int32).reshape(max_batch, max_groups)
        self.group_table = torch.from_numpy(gt).to(dev)
        if rotation is None:
            rotation = random_rotation(seed, head_dim)
        pi, pi_t = rotation
        cent, bnd = value_codebook(value_bits, head_dim)
        self.pi = torch.from_numpy(np.ascontiguousarray(pi, np.float32)).to(dev)
        self.pi_t = torch.from_numpy(np.ascontiguousarray(pi_t, np.float32)).to(dev)
        self.vcent = torch.from_numpy(cent).to(dev)
        self.vbnd = torch.from_numpy(bnd).to(dev)
        # "bias": the zero point of group g, whose block starts at token g * G
        # (turboquant_pro/per_channel_kv.py:245-267 with position_start = g * G)
        self.zp_mean = None
        if zero_point == "bias":
            zp = np.stack([rope_averaged_bias(self.k_bias, rope_theta, head_dim, g * G, G)
                           for g in range(max_groups)])
            self.zp_mean = torch.from_numpy(np.ascontiguousarray(zp, np.float32)).to(dev)
        self.ptrs = N.CachePtrs(
            kcodes=self.kcodes.data_ptr(), vcodes=self.vcodes.data_ptr(),
            vnorm=self.vnorm.data_ptr(), gscale=self.gscale.data_ptr(),
            gmean=self.gmean.data_ptr(), ocount=self.ocount.data_ptr(),
            oent=self.oent.data_ptr(), hot_k=self.hot_k.data_ptr(), hot_v=self.hot_v.data_ptr(),
            block_table=self.block_table.data_ptr(), group_table=self.group_table.data_ptr(),
            pi=self.pi.data_ptr(), pi_t=self.pi_t.data_ptr(), vcent=self.vcent.data_ptr(),
            vbnd=self.vbnd.data_ptr(),
            zp_mean=self.zp_mean.data_ptr() if self.zp_mean is not None else None,
            knorm=self.knorm.data_ptr() if self.knorm is not None else None)
        self.lengths = [0] * max_batch
        self.seq_lens = torch.zeros(max_batch, dtype=i32, device=dev)
        self._overflow = torch.zeros(1, dtype=i32, device=dev)
        # (event, pinned flag word) of appends whose encode flags are not read yet
        self._pending = []
        # the first flagged encode error: sticky until reset(), so every later
        # call that reads the cache raises it, not only the first
        self._error = None
        self._ws = None

    # ------------------------------------------------------------------ #
    @staticmethod
    def _clustered_table(max_batch: int, max_pages: int, P: int, G: int) -> np.ndarray:
        """Default block table.  With 32-token pages, the pages of 8 consecutive
        groups of a sequence form a cluster in which block k of group 8c + w
        sits at page 8k + w: the decode's 8 waves stream groups w = 0..7 of a
        cluster side by side, so their concurrent block reads are adjacent in
        HBM.  Otherwise the identity mapping."""
        bt = np.arange(max_batch * max_pages, dtype=np.int32).reshape(max_batch, max_pages)
        if P != 32 or G % 32 != 0:
            return bt
        nb = G // 32                                # blocks per group
        lp = np.arange(max_pages)                   # logical page = token block
        g, k = lp // nb, lp % nb
        phys = (g // 8) * (8 * nb) + k * 8 + (g % 8)
        return (np.arange(max_batch)[:, None] * max_pages + phys[None, :]).astype(np.int32)

    def _stream(self):
        return ctypes.c_void_p(_torch().cuda.current_stream(self.device).cuda_stream)

    def n_groups(self, b: int) -> int:
        return n_groups_for(self.lengths[b], self.hot_window)

    def hot_length(self, b: int) -> int:
        return self.lengths[b] - self.n_groups(b) * self.group_tokens

    def reset(self) -> None:
        # the cache's contents go, and with them any flags still unread and
        # any error they raised
        self._pending = []
        self._error = None
        self.lengths = [0] * self.max_batch
        self.seq_lens.zero_()

    def check(self, wait: bool = True) -> None:
        """Raise the first error an earlier append's encode flagged (a value
        norm beyond the decode's range, a side-list beyond ``outlier_cap``).
        ``append`` copies the flags to pinned host memory without waiting, so
        that consecutive appends keep the GPU busy; they are read here: by the
        next append (flags already arrived), and with ``wait`` by every call
        that reads the cache (decode, export, dequant, growth).  An error is
        sticky: once flagged, every later check raises it again, because the
        codes that caused it stay in the pool; ``reset`` clears the contents
        and the error.  Under HIP graph capture a host wait is impossible, so
        a capture with flags still unread raises instead of waiting (call
        ``check()`` before capturing)."""
        if self._error is not None:
            raise self._error[0](self._error[1])
        if self._pending and wait and _torch().cuda.is_current_stream_capturing():
            raise RuntimeError("TQKVPool: encode flags of earlier appends are unread; call "
                               "pool.check() before capturing a decode in a HIP graph")
        keep = []
        for ev, flag in self._pending:
            if not wait and not ev.query():
                keep.append((ev, flag))
                continue
            ev.synchronize()
            ovf = int(flag[0])
            if ovf & 2:
                self._pending = []
                self._error = (ValueError, "a value vector's norm exceeds 16376, the largest the "
                               "gfx950 decode carries (softmax weight <= 4 times the norm in fp16)")
            elif ovf & 1:
                self._pending = []
                self._error = (RuntimeError, "outlier side-list exceeded outlier_cap for a group; "
                               "rebuild the pool with a larger outlier_cap")
            if self._error is not None:
                raise self._error[0](self._error[1])
        self._pending = keep

    def grown(self, max_seq_len: int) -> "TQKVPool":
        """A pool of the same format holding up to ``max_seq_len`` tokens per
        sequence, with this pool's contents: every sequence's pages copied
        through both block tables, its group slots and its hot ring (the
        codes are moved, never re-encoded).  Pools with a caller's block
        table cannot grow."""
        torch = _torch()
        self.check()
        if self._custom_table:
            raise ValueError("a pool with a caller's block table cannot grow")
        if max_seq_len <= self.max_seq_len:
            return self
        new = TQKVPool(max_seq_len=max_seq_len, rotation=(self.pi.cpu().numpy(), self.pi_t.cpu().numpy()),
                       **self._init_args)
        if new.oent.shape[2] < self.oent.shape[2]:
            raise ValueError("the grown pool's outlier_cap is smaller")
        B, mp_old, mg_old = self.max_batch, self.max_pages, self.max_groups
        dev = self.device
        old_bt = self.block_table.long()[:, :mp_old]
        new_bt = new.block_table.long()[:, :mp_old]
        src, dst = old_bt.reshape(-1), new_bt.reshape(-1)
        for name in ("kcodes", "vcodes", "vnorm") + (("knorm",) if self.knorm is not None else ()):
            getattr(new, name)[:, dst] = getattr(self, name)[:, src]
        so = self.group_table.long()[:, :mg_old].reshape(-1)
        sn = new.group_table.long()[:, :mg_old].reshape(-1)
        new.gscale[sn] = self.gscale[so]
        new.gmean[sn] = self.gmean[so]
        new.ocount[sn] = self.ocount[so]
        new.oent[sn, :, :self.oent.shape[2]] = self.oent[so]
        new.hot_k.copy_(self.hot_k)
        new.hot_v.copy_(self.hot_v)
        new.lengths = list(self.lengths)
        new.seq_lens.copy_(self.seq_lens)
        torch.cuda.synchronize(dev)
        return new

    # ------------------------------------------------------------------ #
    def append(self, k, v, n_new=None, check_overflow: bool = True) -> None:
        """Append tokens: ``k``, ``v`` ``(max_batch, Hkv, T, D)`` on the device,
        fp16 (fp32 for an fp32 pool); sequence ``b`` takes its first
        ``n_new[b]`` tokens (all T by default).  Equivalent to T one-token ``TurboQuantKVCache.append`` calls
        per sequence (turboquant_pro/core.py:986-1038)."""
        torch = _torch()
        self.check(wait=False)
        B, T = self.max_batch, int(k.shape[2])
        if tuple(k.shape) != (B, self.n_kv_heads, T, self.head_dim) or k.shape != v.shape:
            raise ValueError(f"append expects ({B}, {self.n_kv_heads}, T, {self.head_dim}) K and V")
        if k.dtype != self.dtype or v.dtype != self.dtype:
            raise ValueError(f"append expects {self.input_dtype} keys and values")
        k = k.contiguous()
        v = v.contiguous()
        n_new = [T] * B if n_new is None else [int(x) for x in n_new]
        if len(n_new) != B or min(n_new) < 0 or max(n_new) > T:
            raise ValueError("n_new must give 0 <= n <= T for every sequence")
        prev = list(self.lengths)
        new = [p + n for p, n in zip(prev, n_new)]
        if max(new) > self.max_seq_len:
            raise ValueError(f"sequence length {max(new)} exceeds max_seq_len={self.max_seq_len}")
        items = []
        for b in range(B):
            for g in range(n_groups_for(prev[b], self.hot_window), n_groups_for(new[b], self.hot_window)):
                items += [b, g]
        hot_start = [n_groups_for(L, self.hot_window) * self.group_tokens for L in new]
        # pinned and asynchronous: the caching host allocator keeps the block
        # until the copy, queued behind earlier work on the stream, has run
        host = torch.tensor(prev + n_new + hot_start + items, dtype=torch.int32).pin_memory()
        dev = host.to(self.device, non_blocking=True)
        prev_d, nnew_d, hs_d = dev[:B], dev[B:2 * B], dev[2 * B:3 * B]
        items_d = dev[3 * B:]
        L = N.lib()
        st = self._stream()
        if items:
            self._overflow.zero_()
            N.check(L.tqk_encode_groups(ctypes.byref(self.desc), ctypes.byref(self.ptrs), B,
                                        len(items) // 2, items_d.data_ptr(), prev_d.data_ptr(),
                                        k.data_ptr(), v.data_ptr(), T,
                                        self._overflow.data_ptr(), st), "tqk_encode_groups")
            if check_overflow:
                flag = torch.empty(1, dtype=torch.int32, pin_memory=True)
                flag.copy_(self._overflow, non_blocking=True)
                ev = torch.cuda.Event()
                ev.record(torch.cuda.current_stream(self.device))
                self._pending.append((ev, flag))
        if T > 0:
            N.check(L.tqk_append_hot(ctypes.byref(self.desc), ctypes.byref(self.ptrs), B,
                                     prev_d.data_ptr(), nnew_d.data_ptr(), hs_d.data_ptr(),
                                     k.data_ptr(), v.data_ptr(), T, st), "tqk_append_hot")
        self.lengths = new
        torch.add(prev_d, nnew_d, out=self.seq_lens)

    # ------------------------------------------------------------------ #
    def workspace(self, batch: int, max_len: int):
        torch = _torch()
        need = N.lib().tqk_decode_workspace_bytes(ctypes.byref(self.desc), batch, max_len)
        if self._ws is None or self._ws.numel() < need:
            # zero-filled once: the arrival counters of the in-kernel merge
            # start at zero and every call leaves them there
            self._ws = torch.zeros(int(need), dtype=torch.uint8, device=self.device)
        return self._ws, int(need)

    def _check_q(self, q):
        torch = _torch()
        B = self.max_batch
        if tuple(q.shape) != (B, self.n_q_heads, self.head_dim) or q.dtype != self.dtype:
            raise ValueError(f"decode expects {self.input_dtype} q of shape "
                             f"({B}, {self.n_q_heads}, {self.head_dim})")
        if min(self.lengths) <= 0:
            raise RuntimeError("cache is empty")
        return q.contiguous()

    def decode(self, q, out=None):
        """One decode step for every sequence: ``q`` ``(B, Hq, D)`` (fp16, or
        fp32 for an fp32 pool) ->
        fp32 ``(B, Hq, D)`` attention output over each sequence's whole cache."""
        torch = _torch()
        q = self._check_q(q)
        self.check()
        B, max_len = self.max_batch, max(self.lengths)
        if out is None:
            out = torch.empty((B, self.n_q_heads, self.head_dim), dtype=torch.float32, device=self.device)
        ws, need = self.workspace(B, max_len)
        N.check(N.lib().tqk_decode(ctypes.byref(self.desc), ctypes.byref(self.ptrs), B,
                                   q.data_ptr(), self.seq_lens.data_ptr(), max_len, out.data_ptr(),
                                   ws.data_ptr(), need, self._stream()), "tqk_decode")
        return out

    def decode_partials(self, q):
        """Unnormalised online-softmax state ``(m, l, acc)`` of one decode step:
        ``(B, Hq)``, ``(B, Hq)``, ``(B, Hq, D)`` fp32 with ``out = acc / l``."""
        torch = _torch()
        q = self._check_q(q)
        self.check()
        B, max_len = self.max_batch, max(self.lengths)
        m = torch.empty((B, self.n_q_heads), dtype=torch.float32, device=self.device)
        l_ = torch.empty_like(m)
        acc = torch.empty((B, self.n_q_heads, self.head_dim), dtype=torch.float32, device=self.device)
        ws, need = self.workspace(B, max_len)
        N.check(N.lib().tqk_decode_partials(ctypes.byref(self.desc), ctypes.byref(self.ptrs), B,
                                            q.data_ptr(), self.seq_lens.data_ptr(), max_len,
                                            m.data_ptr(), l_.data_ptr(), acc.data_ptr(),
                                            ws.data_ptr(), need, self._stream()),
                "tqk_decode_partials")
        return m, l_, acc

    # ------------------------------------------------------------------ #
    def dequant_groups(self, items):
        """fp32 reconstructions of groups ``[(b, g), ...]``: keys and values,
        each ``(n, Hkv, G, D)`` (PerChannelKV.decompress / TurboQuantKV.decompress)."""
        torch = _torch()
        self.check()
        n = len(items)
        G, H, D = self.group_tokens, self.n_kv_heads, self.head_dim
        kout = torch.empty((n, H, G, D), dtype=torch.float32, device=self.device)
        vout = torch.empty_like(kout)
        if n:
            it = torch.tensor([x for bg in items for x in bg], dtype=torch.int32).to(self.device)
            N.check(N.lib().tqk_dequant_groups(ctypes.byref(self.desc), ctypes.byref(self.ptrs), n,
                                               it.data_ptr(), kout.data_ptr(), vout.data_ptr(),
                                               self._stream()), "tqk_dequant_groups")
        return kout, vout

    def hot_window_tokens(self, b: int):
        """``(Hkv, n_hot, D)`` keys and values of sequence b's hot window, in the
        pool's input dtype."""
        torch = _torch()
        L, n_cold = self.lengths[b], self.n_groups(b) * self.group_tokens
        idx = torch.arange(n_cold, L, device=self.device) % self.hot_window
        return self.hot_k[b][:, idx], self.hot_v[b][:, idx]

    def _rows(self, b: int, g: int):
        torch = _torch()
        t = torch.arange(g * self.group_tokens, (g + 1) * self.group_tokens, device=self.device)
        phys = self.block_table[b][t // self.page_tokens].long()
        return phys, (t % self.page_tokens)

    def export_group(self, b: int, g: int) -> dict:
        """Group ``g`` of sequence ``b`` in the reference container layout:
        ``kpacked`` (CompressedPerChannelKV.indices), ``nf4_scale``/``nf4_mean``
        ``(H, D)``, ``outlier_idx`` int32 / ``outlier_val`` fp16 (flat over
        ``(1, H, G, D)``), ``vpacked`` (CompressedKV.indices), ``vnorms`` ``(H, G)``.
        PolarQuant keys: ``kpacked`` is the keys' CompressedKV.indices (the value
        pack) and ``knorms`` ``(H, G)`` their norms, with no scale, mean or
        side-list."""
        self.check()
        phys, off = self._rows(b, g)
        H, G, D = self.n_kv_heads, self.group_tokens, self.head_dim
        kp = self.kcodes[:, phys, off].contiguous().cpu().numpy()  # (H, G, D * key_bits / 8)
        vp = self.vcodes[:, phys, off].contiguous().cpu().numpy()  # (H, G, vrow)
        if self.tiled:
            vp = np.stack([pack_values(untile_value_rows(vp[h], self.value_bits, D), self.value_bits)
                           for h in range(H)])
        vn = self.vnorm[:, phys, off].contiguous()
        if self.key_grid == "polar":
            codes = codes_from_key_rows(kp.reshape(H * G, -1), self.key_bits, D)
            return {
                "kpacked": pack_values(codes, self.key_bits).reshape(-1),
                "knorms": self.knorm[:, phys, off].contiguous().cpu().numpy(),
                "position_start": g * G,
                "vpacked": np.ascontiguousarray(vp).reshape(-1),
                "vnorms": vn.cpu().numpy(),
            }
        slot = int(self.group_table[b, g])
        cnt = self.ocount[slot, :, -1].cpu().numpy()
        ent = self.oent[slot].cpu().numpy().view(np.uint32)
        idx, val = [], []
        for h in range(H):
            e = ent[h, :min(int(cnt[h]), ent.shape[1])]
            idx.append((e & 0xFFFF).astype(np.int64) + h * G * D)
            val.append((e >> 16).astype(np.uint16))
        oidx = np.concatenate(idx) if idx else np.zeros(0, np.int64)
        oval = np.concatenate(val).view(np.float16) if val else np.zeros(0, np.float16)
        scale, mean = self.gscale[slot].cpu().numpy(), self.gmean[slot].cpu().numpy()
        # the reference's codes: the stored rows, with the code of the stored
        # fp16 value put back at every outlier position (an fp32 pool stores
        # the reference's codes there already), in the reference's pack
        kb = self.key_bits
        codes = codes_from_key_rows(kp.reshape(H * G, -1), kb, D).reshape(H, G, D)
        if oidx.size and not self.f32:
            h, t, j = oidx // (G * D), (oidx // D) % G, oidx % D
            v32 = oval.astype(np.float32)
            codes[h, t, j] = (uniform_codes(v32, scale[h, j], mean[h, j], kb) if self.key_grid == "uniform"
                              else nf4_codes(v32, scale[h, j], mean[h, j]))
        kp = pack_key_codes(codes, kb)
        # the reference's stored zero point: every channel's ("calibrated"),
        # the DC channels' ("sparse") or none ("bias": recomputed from the
        # bias; "symmetric": there is none, and the container says
        # "calibrated" with no mean, per_channel_kv.py:354-357)
        stored_mean = (mean[:, self.dc_mask] if self.zero_point == "sparse"
                       else None if self.zero_point in ("bias", "symmetric") else mean)
        return {
            "kpacked": kp.reshape(-1),
            "nf4_scale": scale,
            "nf4_mean": stored_mean,
            "zp_mode": "calibrated" if self.zero_point == "symmetric" else self.zero_point,
            "position_start": g * G,
            "outlier_idx": oidx.astype(np.int32),
            "outlier_val": oval,
            "outlier_count": cnt.astype(np.int64),
            "vpacked": np.ascontiguousarray(vp).reshape(-1),
            "vnorms": vn.cpu().numpy(),
        }

    def import_group(self, b: int, g: int, keys: dict | None = None, values: dict | None = None) -> None:
        """Write group ``g`` of sequence ``b`` from the reference container
        layout (the inverse of :meth:`export_group`).  ``keys``: ``kpacked``
        (H*G*D/2 bytes), ``nf4_scale``/``nf4_mean`` (H, D), ``outlier_idx``
        (flat over (H, G, D), token-major within a head as the reference emits
        them) and ``outlier_val`` fp16, or ``None`` outliers (PolarQuant keys:
        ``kpacked``, the value pack of H*G*D codes, and ``knorms`` (H, G)); ``values``:
        ``vpacked`` (reference pack of H*G*D codes) and ``vnorms`` (H, G); a
        tiled pool stores them in its MFMA-tiled order."""
        torch = _torch()
        H, G, D = self.n_kv_heads, self.group_tokens, self.head_dim
        phys, off = self._rows(b, g)
        slot = int(self.group_table[b, g])
        if keys is not None and self.key_grid == "polar":
            kb = self.key_bits
            kp = np.asarray(keys["kpacked"], np.uint8).reshape(-1)
            need = -(-H * G * D * kb // 8)
            if kp.size < need:
                raise ValueError(f"kpacked holds {kp.size} bytes; a group of {kb}-bit keys takes {need}")
            codes = unpack_values(kp, H * G * D, kb).reshape(H * G, D)
            rows = key_rows_from_codes(codes, kb).reshape(H, G, -1)
            self.kcodes[:, phys, off] = torch.from_numpy(np.ascontiguousarray(rows)).to(self.device)
            self.knorm[:, phys, off] = torch.from_numpy(
                np.asarray(keys["knorms"], np.float32).reshape(H, G)).to(self.device)
            # the identity per-channel stats and an empty side-list, as the encode writes them
            self.gscale[slot] = 1.0
            self.gmean[slot] = 0.0
            self.ocount[slot] = 0
        elif keys is not None:
            kb = self.key_bits
            kp = np.asarray(keys["kpacked"], np.uint8).reshape(-1)
            if kp.size != H * G * D * kb // 8:
                raise ValueError(f"kpacked holds {kp.size} bytes; a group of {kb}-bit keys takes "
                                 f"{H * G * D * kb // 8}")
            oidx = keys.get("outlier_idx")
            oval = keys.get("outlier_val")
            oidx = np.zeros(0, np.int64) if oidx is None else np.asarray(oidx, np.int64).reshape(-1)
            oval = np.zeros(0, np.float16) if oval is None else np.asarray(oval, np.float16).reshape(-1)
            if oidx.size != oval.size:
                raise ValueError("outlier_idx and outlier_val differ in length")
            if oidx.size and (oidx.min() < 0 or oidx.max() >= H * G * D):
                raise ValueError("outlier_idx outside the (H, G, D) block")
            # stored form: the zero-level code at every outlier position (fp32
            # pools keep the reference's codes), in the pool's row layout
            codes = unpack_key_codes(kp, H * G * D, kb).reshape(H, G, D)
            if oidx.size and not self.f32:
                zc = 0 if self.key_grid == "uniform" else NF4_ZERO_CODE
                codes[oidx // (G * D), (oidx // D) % G, oidx % D] = zc
            kp = key_rows_from_codes(codes.reshape(H * G, D), kb).reshape(H, G, -1)
            self.kcodes[:, phys, off] = torch.from_numpy(np.ascontiguousarray(kp)).to(self.device)
            self.gscale[slot] = torch.from_numpy(np.asarray(keys["nf4_scale"], np.float32).reshape(H, D)).to(self.device)
            if self.zero_point == "bias":
                self.gmean[slot] = self.zp_mean[g]
            elif self.zero_point == "symmetric":
                self.gmean[slot] = 0.0
            elif self.zero_point == "sparse":
                full = np.zeros((H, D), np.float32)
                full[:, self.dc_mask] = np.asarray(keys["nf4_mean"], np.float32).reshape(H, -1)
                self.gmean[slot] = torch.from_numpy(full).to(self.device)
            else:
                self.gmean[slot] = torch.from_numpy(np.asarray(keys["nf4_mean"], np.float32).reshape(H, D)).to(self.device)
            h = oidx // (G * D)
            pos = oidx % (G * D)  # token * D + channel within the head
            cap = self.oent.shape[2]
            ent = np.zeros((H, cap), np.uint32)
            cnt = np.zeros((H, 8), np.int32)
            for hh in range(H):
                m = h == hh
                ph = pos[m]
                if ph.size > (cap if self.desc.outlier_cap > 0 else 0):
                    raise ValueError("more outliers in a head than the pool's outlier_cap")
                if ph.size > 1 and np.any(np.diff(ph) <= 0):
                    raise ValueError("outliers of a head must be in ascending token-major order")
                vals = oval[m].view(np.uint16).astype(np.uint32)
                ent[hh, :ph.size] = ph.astype(np.uint32) | (vals << np.uint32(16))
                tok = ph // D
                for k in range(8):
                    cnt[hh, k] = int(np.count_nonzero(tok < 32 * (k + 1)))
            self.oent[slot] = torch.from_numpy(ent.view(np.int32)).to(self.device)
            self.ocount[slot] = torch.from_numpy(cnt).to(self.device)
        if values is not None:
            vrow = D * self.value_bits // 8
            if self.tiled:
                codes = unpack_values(np.asarray(values["vpacked"], np.uint8), H * G * D,
                                      self.value_bits).reshape(H, G, D)
                vp = np.stack([tile_value_rows(codes[hh], self.value_bits) for hh in range(H)])
            else:
                vp = np.asarray(values["vpacked"], np.uint8)[: H * G * vrow].reshape(H, G, vrow)
            self.vcodes[:, phys, off] = torch.from_numpy(np.ascontiguousarray(vp)).to(self.device)
            self.vnorm[:, phys, off] = torch.from_numpy(
                np.asarray(values["vnorms"], np.float32).reshape(H, G)).to(self.device)

    def load_sequence(self, b: int, groups, hot_k, hot_v) -> None:
        """Restore sequence ``b`` (empty) from coded groups and hot tokens:
        ``groups`` = ``[(keys, values), ...]`` in :meth:`import_group`'s
        layout, written as they are (no re-encode), then ``hot_k``/``hot_v``
        ``(Hkv, n_hot, D)`` into the hot ring (in the pool's input dtype).  The split must be the
        flush cadence's: ``n_groups_for(len(groups) * G + n_hot)`` is
        ``len(groups)``."""
        torch = _torch()
        if self.lengths[b] != 0:
            raise ValueError(f"sequence {b} is not empty")
        G, W = self.group_tokens, self.hot_window
        n_hot = int(hot_k.shape[1])
        L = len(groups) * G + n_hot
        if tuple(hot_k.shape) != (self.n_kv_heads, n_hot, self.head_dim) or hot_v.shape != hot_k.shape:
            raise ValueError(f"hot tokens must be ({self.n_kv_heads}, n, {self.head_dim}) keys and values")
        if n_groups_for(L, W) != len(groups) or L > self.max_seq_len:
            raise ValueError(f"{len(groups)} groups + {n_hot} hot tokens is not a state of the "
                             f"flush cadence (hot window {W}, group {G}) within {self.max_seq_len} tokens")
        for g, (keys, values) in enumerate(groups):
            self.import_group(b, g, keys=keys, values=values)
        if n_hot:
            idx = torch.arange(L - n_hot, L, device=self.device) % W
            self.hot_k[b][:, idx] = hot_k.to(device=self.device, dtype=self.dtype)
            self.hot_v[b][:, idx] = hot_v.to(device=self.device, dtype=self.dtype)
        self.lengths[b] = L
        self.seq_lens[b] = L
