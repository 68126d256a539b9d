"""KVCache: drop-in for ``modelcore.cache.KVCache`` (modelcore/cache.py:13-119).

Same constructor, attributes, methods and assertion messages. K and V live in two preallocated
tensors of shape (n_slots, B, T_max, H_kv, D) in the compute dtype, zero-filled at creation
(modelcore/cache.py:22-23): one token's K (or V) for all KV heads is a contiguous H_kv*D run,
1 KiB at H_kv=4, D=128 in bf16, which is the unit the HIP append and decode kernels move.
``cache_seqlens`` is the per-row position on the device (int32), and ``_pos_uniform`` its host
mirror (the shared position, or None once rows are right-ragged).

One attribute is added to the reference's: ``shared_prefix``, the number of leading positions at
which every row holds the same K/V (after ``prefill`` of one prompt into all rows), which the
decode operator can exploit (``flash_attn_with_kvcache(..., shared_prefix=...)``).

The copies of ``prefill`` and ``prefill_row`` run the HIP replication kernel
(``mcamd_kv_replicate``); the appends happen inside the attention operator
(``modelcore_amd.kernels.flash_attn``). Position bookkeeping (``advance``, ``reset``) stays on
torch, as in the reference.
"""
from __future__ import annotations

import torch

from modelcore_amd import _ext


class KVCache:
    def __init__(self, batch_size, n_kv_head, seq_len, head_dim, num_kv_slots, device, dtype):
        self.batch_size = batch_size
        self.max_seq_len = seq_len
        self.n_slots = num_kv_slots
        self.n_kv_head = n_kv_head
        self.head_dim = head_dim
        # (n_slots, B, T, H, D); fewer slots than layers when layers share a KV slot.
        self.k_cache = torch.zeros(num_kv_slots, batch_size, seq_len, n_kv_head, head_dim,
                                   device=device, dtype=dtype)
        self.v_cache = torch.zeros(num_kv_slots, batch_size, seq_len, n_kv_head, head_dim,
                                   device=device, dtype=dtype)
        # Position of each row (int32 on the device), read by the attention kernels.
        self.cache_seqlens = torch.zeros(batch_size, dtype=torch.int32, device=device)
        # Host mirror: the shared position of every row, or None once rows are right-ragged.
        # Maintained without reading cache_seqlens back, so decode never syncs the host.
        self._pos_uniform = 0
        # Non-KV per-row state (recurrent/smear state); every tensor is (batch, ...).
        self.state = {}
        # Positions [0, shared_prefix) of every row hold copies of row 0's K/V (prefill() of one
        # prompt into all rows); the decode operator may then read them from row 0 for every row.
        # Not in the reference: set by prefill(), cleared by reset() and the per-row prefills.
        self.shared_prefix = 0

    def reset(self):
        """Back to empty. K/V are deliberately not zeroed: a row only ever reads keys at indices
        <= its own position, all of which it wrote itself (modelcore/cache.py:38-45)."""
        self.cache_seqlens.zero_()
        self.state = {}
        self._pos_uniform = 0
        self.shared_prefix = 0

    def get_pos(self):
        """The single position every row is at; raises on a right-ragged cache."""
        assert self._pos_uniform is not None, \
            "get_pos() on a right-ragged KV cache; read cache_seqlens or check uniform_pos()"
        return self._pos_uniform

    def uniform_pos(self):
        """get_pos() without the assert: the shared position, or None if the cache is ragged."""
        return self._pos_uniform

    def get_slot_cache(self, slot):
        """(k_cache, v_cache) views of one KV slot, each (B, T_max, H_kv, D)."""
        return self.k_cache[slot], self.v_cache[slot]

    def advance(self, num_tokens):
        """Advance every row by num_tokens. Keeps ragged rows' differences unchanged, which is all
        raggedness is (modelcore/cache.py:62-73)."""
        self.cache_seqlens += num_tokens
        self.note_device_advance(num_tokens)

    def note_device_advance(self, num_tokens):
        """Move the host mirror of the positions after an operator call that already advanced
        cache_seqlens on the device (flash_attn_with_kvcache(..., advance=num_tokens)): the two
        together are advance(num_tokens)."""
        if self._pos_uniform is not None:
            self._pos_uniform += num_tokens

    def _replicate_from(self, other, row_begin, n_rows, n_tokens, src_row=0):
        """HIP copy of row `src_row`, positions [0, n_tokens), of every slot of `other` into rows
        [row_begin, row_begin + n_rows) of this cache."""
        _ext.require_rocm(self.k_cache, other.k_cache, what="KVCache replication")
        if self.k_cache.dtype != other.k_cache.dtype:
            raise TypeError(f"cache dtypes differ: {self.k_cache.dtype} vs {other.k_cache.dtype}")
        if self.k_cache.device != other.k_cache.device:
            raise ValueError(f"caches on different devices: {self.k_cache.device} vs "
                             f"{other.k_cache.device}")
        if self.n_slots == 0 or n_rows == 0 or n_tokens == 0:
            return
        row_elems = self.n_kv_head * self.head_dim
        lib = _ext.lib()
        assert 0 <= src_row < other.batch_size, f"source row {src_row} out of range"
        src_off = src_row * other.k_cache.stride(1) * other.k_cache.element_size()
        st = lib.mcamd_kv_replicate(
            other.k_cache.data_ptr() + src_off, other.v_cache.data_ptr() + src_off,
            self.k_cache.data_ptr(),
            self.v_cache.data_ptr(), self.n_slots, other.k_cache.stride(0),
            self.k_cache.stride(0), self.batch_size, self.k_cache.stride(1), row_begin, n_rows,
            n_tokens, row_elems,
            _ext.dtype_code(self.k_cache.dtype), _ext.stream_handle(self.k_cache.device))
        _ext.check(st, "kv_replicate")

    def _assert_same_geometry(self, other):
        geometry = lambda c: (c.n_slots, c.n_kv_head, c.head_dim)
        assert geometry(self) == geometry(other), \
            f"cache geometry (slots, H_kv, D) differs: {geometry(self)} vs {geometry(other)}"

    def prefill(self, other):
        """Copy a batch=1 prefilled cache into every row (modelcore/cache.py:75-90): one prompt
        prefilled once, then decoded as many samples in parallel."""
        assert self.get_pos() == 0, "Cannot prefill a non-empty KV cache"
        self._assert_same_geometry(other)
        assert other.max_seq_len <= self.max_seq_len, "source cache is longer than this one"
        other_pos = other.get_pos()
        self._replicate_from(other, 0, self.batch_size, other_pos)
        self.cache_seqlens.fill_(other_pos)
        self._pos_uniform = other_pos
        self.shared_prefix = other_pos  # every row (row 0 included) now holds the same prompt
        # Expand any batch=1 extra state to every row.
        for key, value in other.state.items():
            self.state[key] = value.expand(self.batch_size, *([-1] * (value.dim() - 1))).clone()

    def prefill_rows(self, other, lengths, num_samples=1):
        """Copy the prompts of a cache prefilled together -- row p of `other` holds prompt p,
        right-padded to the longest -- into rows [p * num_samples, (p + 1) * num_samples), each
        ending at its prompt's length (right-ragged). The batched counterpart of calling
        prefill_row once per prompt and sample (modelcore/cache.py:92-119), without its host
        reads: the lengths are given. Positions past a row's length hold the padding's K/V, which
        attention never reads (they lie beyond cache_seqlens) and decode overwrites."""
        lengths = [int(n) for n in lengths]
        assert other.batch_size == len(lengths), "one source row per prompt length"
        assert self.batch_size == len(lengths) * num_samples, \
            f"batch_size {self.batch_size} != {len(lengths)} prompts x {num_samples} samples"
        assert self.get_pos() == 0, "Cannot prefill a non-empty KV cache"
        self._assert_same_geometry(other)
        assert not other.state, "per-row extra state is not carried by the batched prefill"
        for p, n in enumerate(lengths):
            assert 0 < n <= other.max_seq_len, f"prompt length {n} out of range"
            assert n <= self.max_seq_len, f"prompt of {n} tokens exceeds cache length {self.max_seq_len}"
            self._replicate_from(other, p * num_samples, num_samples, n, src_row=p)
        per_row = [n for n in lengths for _ in range(num_samples)]
        self.cache_seqlens.copy_(torch.tensor(per_row, dtype=torch.int32))
        self._pos_uniform = per_row[0] if len(set(per_row)) == 1 else None
        self.shared_prefix = lengths[0] if len(lengths) == 1 else 0  # one prompt: all rows alike

    def fill_sample_rows(self, lengths, num_samples):
        """After a packed prefill wrote prompt p into row p * num_samples (PackedPrefill), copy it
        into that prompt's other sample rows [p * num_samples + 1, (p + 1) * num_samples) and set
        every row's position to its prompt's length -- what the reference's prefill_row does per
        prompt and sample (modelcore/cache.py:92-119), without its host reads: the lengths are
        given. One prompt leaves every row alike (shared_prefix)."""
        lengths = [int(n) for n in lengths]
        assert self.batch_size == len(lengths) * num_samples, \
            f"batch_size {self.batch_size} != {len(lengths)} prompts x {num_samples} samples"
        for p, n in enumerate(lengths):
            assert 0 < n <= self.max_seq_len, f"prompt of {n} tokens exceeds cache length {self.max_seq_len}"
            if num_samples > 1:
                self._replicate_from(self, p * num_samples + 1, num_samples - 1, n,
                                     src_row=p * num_samples)
        per_row = [n for n in lengths for _ in range(num_samples)]
        self.cache_seqlens.copy_(torch.tensor(per_row, dtype=torch.int32))
        self._pos_uniform = per_row[0] if len(set(per_row)) == 1 else None
        self.shared_prefix = lengths[0] if len(lengths) == 1 else 0

    def prefill_row(self, row, other):
        """Copy a batch=1 prefilled cache into row `row` only (modelcore/cache.py:92-119); rows
        filled this way end at different positions (right-ragged)."""
        assert other.batch_size == 1, "prefill_row copies from a batch=1 cache"
        assert 0 <= row < self.batch_size, f"row {row} out of range for batch_size {self.batch_size}"
        assert self.cache_seqlens[row].item() == 0, "Cannot prefill a non-empty KV cache row"
        self._assert_same_geometry(other)
        other_pos = other.get_pos()
        assert other_pos <= self.max_seq_len, f"prompt of {other_pos} tokens exceeds cache length {self.max_seq_len}"
        self._replicate_from(other, row, 1, other_pos)
        self.cache_seqlens[row] = other_pos
        self.shared_prefix = 0  # rows may now hold different prompts
        # Per-row extra state: a zero buffer per key, shaped from the source, filled row by row.
        for key, value in other.state.items():
            if key not in self.state:
                self.state[key] = value.new_zeros((self.batch_size, *value.shape[1:]))
            self.state[key][row] = value[0]
        # Uniform again only when every row sits at the same position (e.g. equal prompts).
        positions = set(self.cache_seqlens.tolist())
        self._pos_uniform = positions.pop() if len(positions) == 1 else None


class PackedPrefill:
    """Several prompts prefilled together into chosen rows of a KVCache, their tokens packed one
    after another along a single sequence axis: ``model(idx, kv_cache=PackedPrefill(...))`` with
    idx (1, total) runs every projection on the real tokens only (no padding), and each attention
    layer appends prompt p's K/V at positions [0, lengths[p]) of row rows[p] and attends there
    (``flash_attn_varlen_with_kvcache``), in place -- no transient cache, no second write. The
    reference prefills each prompt alone into a batch-1 cache and copies it into its row
    (modelcore/generate.py:67-80 -> KVCache.prefill_row, modelcore/cache.py:92-119).

    The rows must be empty (the reference's prefill_row asserts that too); on a cache whose host
    mirror says every row is at 0 this costs no host read. After the forward, each row sits at its
    own prompt's length (``advance``)."""

    shared_prefix = 0

    def __init__(self, cache, rows, lengths):
        rows, lengths = [int(r) for r in rows], [int(n) for n in lengths]
        assert rows and len(rows) == len(lengths), "one cache row per prompt"
        assert len(set(rows)) == len(rows), "rows must be distinct"
        assert all(0 <= r < cache.batch_size for r in rows), \
            f"rows {rows} out of range for batch_size {cache.batch_size}"
        assert min(lengths) > 0, "empty prompt"
        longest = max(lengths)
        assert longest <= cache.max_seq_len, \
            f"prompt of {longest} tokens exceeds cache length {cache.max_seq_len}"
        if cache.uniform_pos() != 0:
            busy = cache.cache_seqlens[rows].tolist()
            assert not any(busy), "Cannot prefill a non-empty KV cache row"
        dev = cache.cache_seqlens.device
        self.cache = cache
        self.row_list, self.lengths = rows, lengths
        cu = [0]
        for n in lengths:
            cu.append(cu[-1] + n)
        self.total, self.max_seqlen = cu[-1], longest
        self.rows = torch.tensor(rows, dtype=torch.int32, device=dev)
        self.cu_seqlens = torch.tensor(cu, dtype=torch.int32, device=dev)
        # Each token's position (its index within its prompt), for RoPE.
        self.positions = torch.cat([torch.arange(n) for n in lengths]).to(dev)
        # Index of each prompt's last token in the packed sequence.
        self.last = torch.tensor(cu[1:], device=dev) - 1

    @property
    def cache_seqlens(self):
        return self.cache.cache_seqlens

    def get_slot_cache(self, slot):
        return self.cache.get_slot_cache(slot)

    def advance(self, num_tokens):
        """Each row moves on by its own prompt's length (one device add, no host read)."""
        assert num_tokens == self.total, "a packed forward covers every prompt's tokens"
        c = self.cache
        c.cache_seqlens.index_add_(0, self.rows.long(),
                                   torch.tensor(self.lengths, dtype=torch.int32,
                                                device=c.cache_seqlens.device))
        every = sorted(self.row_list) == list(range(c.batch_size))
        c._pos_uniform = self.lengths[0] if (c._pos_uniform == 0 and every and
                                             len(set(self.lengths)) == 1) else None
        c.shared_prefix = 0
