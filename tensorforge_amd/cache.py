"""Paged KV cache with transactional appends, writing pages on gfx950.

Host mirror of ``tensorforge/cache/paged.py`` (PagedKVCache and its
dataclasses): the same public names, method signatures, allocation order
(lowest free page and sequence slot first), error types and messages, so the
reference's scheduler and decode executors can use it unchanged.  What
differs is the device work:

* ``write_layer`` is one ``tf_paged_kv_write_range`` launch for any token
  count: the kernel resolves each position through the sequence's
  block-table row, where the reference builds index tensors with three
  launches plus an ``index_put`` per cache (cache/paged.py:212-235);
* block tables and sequence lengths live on the host (the allocator's
  authority) and reach the device with one copy per table, made only when a
  device reader asks (``write_layer``, ``layer_view``, the ``block_tables``
  and ``sequence_lengths`` attributes), where the reference issues one device
  write per table entry and per length update (cache/paged.py:174-175,
  253-258, 268-269, 290-291); a decode step that stages its own tables therefore
  costs the cache no device work at all;
* ``materialize`` gathers with one indexing operation.

Page writes need the cache on a CUDA (HIP) device -- there is no CPU write
path -- but the allocator, reservations and views work for any device.
"""

from __future__ import annotations

import heapq
from dataclasses import dataclass, field

import torch
from torch import Tensor

from tensorforge_amd import _native


class CacheExhaustedError(RuntimeError):
    """An append cannot reserve all the physical pages it needs."""


@dataclass(frozen=True, slots=True)
class CacheStats:
    total_blocks: int
    used_blocks: int
    free_blocks: int
    active_sequences: int
    committed_tokens: int
    reserved_tokens: int


@dataclass(frozen=True, slots=True)
class PagedKVCacheConfig:
    """Geometry of the cache (cache/paged.py:27-60)."""

    num_layers: int
    num_blocks: int
    block_size: int
    num_kv_heads: int
    head_dim: int
    max_sequences: int
    max_sequence_length: int
    dtype: torch.dtype
    device: torch.device

    def __post_init__(self) -> None:
        for name in ("num_layers", "num_blocks", "block_size", "num_kv_heads", "head_dim",
                     "max_sequences", "max_sequence_length"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive")
        if self.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise TypeError(f"unsupported cache dtype: {self.dtype}")
        device = torch.device(self.device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        object.__setattr__(self, "device", device)

    @property
    def max_blocks_per_sequence(self) -> int:
        return -(-self.max_sequence_length // self.block_size)


@dataclass(frozen=True, slots=True)
class AppendReservation:
    request_id: str
    sequence_slot: int
    start_position: int
    token_count: int
    reservation_id: int

    @property
    def end_position(self) -> int:
        return self.start_position + self.token_count


@dataclass(frozen=True, slots=True)
class PagedLayerView:
    key_cache: Tensor
    value_cache: Tensor
    block_table: Tensor
    context_length: int


@dataclass(frozen=True, slots=True)
class CacheAppendLocation:
    physical_block: int
    block_offset: int


@dataclass(frozen=True, slots=True)
class SequenceLayout:
    physical_blocks: tuple[int, ...]
    context_length: int


@dataclass(slots=True)
class _Sequence:
    slot: int
    serial: int
    length: int = 0
    pages: list[int] = field(default_factory=list)
    pending: int | None = None  # id of the open reservation
    truncations: int = 0  # bumped whenever pages are removed from the end


@dataclass(slots=True)
class _Pending:
    reservation: AppendReservation
    new_pages: list[int]
    layers: set[int] = field(default_factory=set)


class PagedKVCache:
    """Physical KV pages with per-request transactional appends
    (cache/paged.py:109-402)."""

    def __init__(self, config: PagedKVCacheConfig, page_order: list[int] | None = None) -> None:
        """``page_order`` (no reference counterpart): the order in which free
        pages are handed out, e.g. a seeded permutation to exercise
        non-contiguous tables; by default the lowest free page first, as in
        the reference."""

        self.config = config
        shape = (config.num_layers, config.num_blocks, config.block_size, config.num_kv_heads,
                 config.head_dim)
        self.key_cache = torch.empty(shape, dtype=config.dtype, device=config.device)
        self.value_cache = torch.empty_like(self.key_cache)
        self._host_tables = torch.full((config.max_sequences, config.max_blocks_per_sequence), -1,
                                       dtype=torch.int32)
        self._host_lengths = torch.zeros(config.max_sequences, dtype=torch.int32)
        self._tables_np = self._host_tables.numpy()
        self._lengths_np = self._host_lengths.numpy()
        if config.device.type == "cpu":
            self._device_tables, self._device_lengths = self._host_tables, self._host_lengths
        else:
            self._device_tables = self._host_tables.to(config.device)
            self._device_lengths = self._host_lengths.to(config.device)
        self._stale = False
        order = list(range(config.num_blocks)) if page_order is None else list(page_order)
        if sorted(order) != list(range(config.num_blocks)):
            raise ValueError("page_order must be a permutation of the page ids")
        self._rank = {page: rank for rank, page in enumerate(order)}
        self._page_of_rank = order
        self._free_pages = list(range(config.num_blocks))  # heap of ranks: next page first
        self._free_slots = list(range(config.max_sequences))
        self._owner: list[str | None] = [None] * config.num_blocks
        self._sequences: dict[str, _Sequence] = {}
        self._pending: dict[int, _Pending] = {}
        self._next_id = 0
        self._next_serial = 0

    # -- device copies of the control state ---------------------------------
    @property
    def block_tables(self) -> Tensor:
        """[max_sequences, max_blocks_per_sequence] int32 on the cache device
        (-1 = unmapped), current as of this call."""

        self._stage()
        return self._device_tables

    @property
    def sequence_lengths(self) -> Tensor:
        """[max_sequences] int32 committed lengths on the cache device."""

        self._stage()
        return self._device_lengths

    def _stage(self) -> None:
        # Pageable source: the copy completes before it returns, so later host
        # edits cannot race it, and it is ordered after earlier device readers
        # on the current stream.
        if self._stale:
            self._device_tables.copy_(self._host_tables)
            self._device_lengths.copy_(self._host_lengths)
            self._stale = False

    # -- allocation -------------------------------------------------------
    def create_sequence(self, request_id: str) -> None:
        if not request_id:
            raise ValueError("request_id must be non-empty")
        if request_id in self._sequences:
            raise ValueError(f"sequence already exists: {request_id}")
        if not self._free_slots:
            raise CacheExhaustedError("no free sequence slots")
        self._sequences[request_id] = _Sequence(slot=heapq.heappop(self._free_slots),
                                                serial=self._next_serial)
        self._next_serial += 1

    def begin_append(self, request_id: str, token_count: int) -> AppendReservation:
        sequence = self._sequence(request_id)
        if token_count <= 0:
            raise ValueError("token_count must be positive")
        if sequence.pending is not None:
            raise RuntimeError("sequence already has an active append")
        end = sequence.length + token_count
        if end > self.config.max_sequence_length:
            raise CacheExhaustedError("append exceeds maximum sequence length")
        needed = -(-end // self.config.block_size) - len(sequence.pages)
        if needed > len(self._free_pages):
            raise CacheExhaustedError(
                f"KV cache needs {needed} blocks but only {len(self._free_pages)} are free"
            )
        new_pages = [self._page_of_rank[heapq.heappop(self._free_pages)]
                     for _ in range(max(needed, 0))]
        for page in new_pages:
            if self._owner[page] is not None:
                raise RuntimeError("allocator ownership corruption detected")
            self._owner[page] = request_id
        first_new = len(sequence.pages)
        sequence.pages.extend(new_pages)
        if new_pages:
            self._write_table(sequence.slot, first_new, new_pages)
        reservation = AppendReservation(request_id, sequence.slot, sequence.length, token_count,
                                        self._next_id)
        self._next_id += 1
        self._pending[reservation.reservation_id] = _Pending(reservation, new_pages)
        sequence.pending = reservation.reservation_id
        return reservation

    # -- page writes --------------------------------------------------------
    def write_layer(self, reservation: AppendReservation, layer_index: int, keys: Tensor,
                    values: Tensor) -> None:
        """Write the reservation's tokens of one layer (cache/paged.py:191-236):
        token t lands at position start + t through the sequence's pages."""

        pending = self._reservation(reservation)
        if not 0 <= layer_index < self.config.num_layers:
            raise IndexError("layer_index is out of range")
        expected = (reservation.token_count, self.config.num_kv_heads, self.config.head_dim)
        for name, tensor in (("keys", keys), ("values", values)):
            if tuple(tensor.shape) != expected:
                raise ValueError(f"{name} must have shape {expected}")
            if tensor.dtype != self.config.dtype or tensor.device != self.config.device:
                raise ValueError(f"{name} must share cache dtype and device")
        if self.config.device.type != "cuda":
            raise ValueError("paged KV writes require CUDA tensors")
        sequence = self._sequence(reservation.request_id)
        keys = keys.contiguous()
        values = values.contiguous()
        key_layer = self.key_cache[layer_index]
        value_layer = self.value_cache[layer_index]
        table = self.block_tables[sequence.slot]
        _native.check(
            _native.library().tf_paged_kv_write_range(
                keys.data_ptr(), values.data_ptr(), key_layer.data_ptr(), value_layer.data_ptr(),
                table.data_ptr(), table.numel(), reservation.start_position,
                reservation.token_count, self.config.num_kv_heads, self.config.head_dim,
                self.config.num_blocks, self.config.block_size,
                _native.dtype_code(self.config.dtype), _native.current_stream(self.config.device),
            ),
            "write_layer",
        )
        pending.layers.add(layer_index)

    def record_layer_write(self, reservation: AppendReservation, layer_index: int) -> None:
        """Mark a layer written by another writer (cache/paged.py:330-338)."""

        pending = self._reservation(reservation)
        if not 0 <= layer_index < self.config.num_layers:
            raise IndexError("layer_index is out of range")
        pending.layers.add(layer_index)

    def record_all_layers_written(self, reservation: AppendReservation) -> None:
        """Mark every layer written at once (no reference counterpart: a
        whole-model decode step writes all layers of its tokens together)."""

        self._reservation(reservation).layers.update(range(self.config.num_layers))

    # -- transactions ---------------------------------------------------------
    def commit(self, reservation: AppendReservation, accepted_tokens: int | None = None) -> None:
        pending = self._reservation(reservation)
        accepted = reservation.token_count if accepted_tokens is None else accepted_tokens
        if not 0 <= accepted <= reservation.token_count:
            raise ValueError("accepted_tokens must be within the reservation")
        if accepted > 0 and len(pending.layers) != self.config.num_layers:
            raise RuntimeError("every cache layer must be written before commit")
        sequence = self._sequence(reservation.request_id)
        sequence.length = reservation.start_position + accepted
        keep = -(-sequence.length // self.config.block_size)
        dropped = sequence.pages[keep:]
        if dropped:
            self._tables_np[sequence.slot, keep:keep + len(dropped)] = -1
            sequence.truncations += 1
            for page in dropped:
                self._owner[page] = None
                heapq.heappush(self._free_pages, self._rank[page])
            del sequence.pages[keep:]
        self._lengths_np[sequence.slot] = sequence.length
        self._stale = True
        sequence.pending = None
        del self._pending[reservation.reservation_id]

    def rollback(self, reservation: AppendReservation) -> None:
        """Abort an append, returning only the pages it allocated."""

        pending = self._reservation(reservation)
        sequence = self._sequence(reservation.request_id)
        first = len(sequence.pages) - len(pending.new_pages)
        if pending.new_pages:
            self._tables_np[sequence.slot, first:len(sequence.pages)] = -1
            self._stale = True
            sequence.truncations += 1
            del sequence.pages[first:]
            for page in pending.new_pages:
                self._owner[page] = None
                heapq.heappush(self._free_pages, self._rank[page])
        sequence.pending = None
        del self._pending[reservation.reservation_id]

    def release(self, request_id: str) -> None:
        """Cancel pending work and return every page and the slot of a request."""

        sequence = self._sequence(request_id)
        if sequence.pending is not None:
            self.rollback(self._pending[sequence.pending].reservation)
        for page in sequence.pages:
            if self._owner[page] != request_id:
                raise RuntimeError("allocator ownership corruption detected")
            self._owner[page] = None
            heapq.heappush(self._free_pages, self._rank[page])
        self._tables_np[sequence.slot] = -1
        self._lengths_np[sequence.slot] = 0
        self._stale = True
        heapq.heappush(self._free_slots, sequence.slot)
        del self._sequences[request_id]

    # -- views ----------------------------------------------------------------
    def block_owners(self) -> tuple[str | None, ...]:
        return tuple(self._owner)

    def sequence_layout(self, request_id: str,
                        reservation: AppendReservation | None = None) -> SequenceLayout:
        """Host-side page list and length; no device synchronisation."""

        sequence = self._sequence(request_id)
        length = self._visible_length(request_id, sequence, reservation)
        return SequenceLayout(tuple(sequence.pages), length)

    def page_list(self, request_id: str) -> tuple[list[int], tuple[int, int]]:
        """The sequence's physical pages in logical order -- the live list,
        which callers must not modify -- and a version key that changes when
        the sequence is recreated or loses pages, so a caller mirroring the
        row can append only the pages added since it last looked (no
        reference counterpart: the decode executor's table staging)."""

        sequence = self._sequence(request_id)
        return sequence.pages, (sequence.serial, sequence.truncations)

    def append_location(self, reservation: AppendReservation,
                        token_offset: int = 0) -> CacheAppendLocation:
        self._reservation(reservation)
        if not 0 <= token_offset < reservation.token_count:
            raise IndexError("token_offset is outside the append reservation")
        sequence = self._sequence(reservation.request_id)
        logical, offset = divmod(reservation.start_position + token_offset, self.config.block_size)
        return CacheAppendLocation(sequence.pages[logical], offset)

    def layer_view(self, request_id: str, layer_index: int,
                   reservation: AppendReservation | None = None) -> PagedLayerView:
        sequence = self._sequence(request_id)
        if not 0 <= layer_index < self.config.num_layers:
            raise IndexError("layer_index is out of range")
        length = self._visible_length(request_id, sequence, reservation)
        return PagedLayerView(self.key_cache[layer_index], self.value_cache[layer_index],
                              self.block_tables[sequence.slot], length)

    def materialize(self, request_id: str, layer_index: int) -> tuple[Tensor, Tensor]:
        """Committed K/V rows of a sequence in logical order."""

        view = self.layer_view(request_id, layer_index)
        sequence = self._sequence(request_id)
        positions = torch.arange(view.context_length)
        pages = torch.tensor(sequence.pages, dtype=torch.int64)[
            positions // self.config.block_size] if view.context_length else positions
        offsets = positions % self.config.block_size
        pages = pages.to(self.config.device)
        offsets = offsets.to(self.config.device)
        return view.key_cache[pages, offsets].clone(), view.value_cache[pages, offsets].clone()

    def stats(self) -> CacheStats:
        return CacheStats(
            total_blocks=self.config.num_blocks,
            used_blocks=self.config.num_blocks - len(self._free_pages),
            free_blocks=len(self._free_pages),
            active_sequences=len(self._sequences),
            committed_tokens=sum(s.length for s in self._sequences.values()),
            reserved_tokens=sum(p.reservation.token_count for p in self._pending.values()),
        )

    # -- internals --------------------------------------------------------------
    def _write_table(self, slot: int, first: int, pages: list[int]) -> None:
        self._tables_np[slot, first:first + len(pages)] = pages
        self._stale = True

    def _visible_length(self, request_id: str, sequence: _Sequence,
                        reservation: AppendReservation | None) -> int:
        if reservation is None:
            return sequence.length
        self._reservation(reservation)
        if reservation.request_id != request_id:
            raise ValueError("reservation belongs to another sequence")
        return reservation.end_position

    def _sequence(self, request_id: str) -> _Sequence:
        try:
            return self._sequences[request_id]
        except KeyError as error:
            raise KeyError(f"unknown sequence: {request_id}") from error

    def _reservation(self, reservation: AppendReservation) -> _Pending:
        try:
            pending = self._pending[reservation.reservation_id]
        except KeyError as error:
            raise RuntimeError("append reservation is no longer active") from error
        if pending.reservation != reservation:
            raise RuntimeError("append reservation identity mismatch")
        return pending
