"""Fused paged KV compression engine (host side of kvmi_kstats/encode/decode_paged).

One call compresses every layer of a request straight from vLLM's paged KV caches:
gather + random-sign FWHT + min-max quantization + bitpack, written into one packed
stream per layer chunk (the reference's 8-layer chunks above 500 MiB,
compression_manager.py:229-235, :365-537), plus bf16 metadata.  Decompression is
the exact inverse and scatters into the caches through the block table.

All work is enqueued on the current torch stream; nothing synchronizes unless the
caller asks for the device error word (``check_errors``).
"""

from __future__ import annotations

import dataclasses

import ctypes
import math
import os
import threading
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib
from .profiles import LayerProfile, rademacher_sign_bits

CHUNK_THRESHOLD_BYTES = 500 * 1024 * 1024  # compression_manager.py:230-231
CHUNK_LAYERS = 8                             # compression_manager.py:235
DEFAULT_SEED = 0x3333                        # kvserve_transformer.py:22


def chunk_ranges(num_layers: int, raw_bytes: int, chunk_layers: int = CHUNK_LAYERS) -> List[Tuple[int, int]]:
    if raw_bytes > CHUNK_THRESHOLD_BYTES:
        return [(s, min(s + chunk_layers, num_layers)) for s in range(0, num_layers, chunk_layers)]
    return [(0, num_layers)]


def _ptr(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else int(t.data_ptr())


def _upload(host: torch.Tensor, device) -> torch.Tensor:
    """Device copy of a host tensor that does not wait for the device: a pinned copy of
    it sent by a non-blocking copy on the current stream (the caching host allocator
    keeps the pinned buffer until that copy has run)."""
    dev = torch.device(device)
    if dev.type != "cuda":
        return host.to(dev)
    return host.pin_memory().to(dev, non_blocking=True)


def _stream_handle() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


DEFAULT_AXES = ("channel", "token")  # (axis_key, axis_value): kvserve_quantizer.py defaults


class _SignCache:
    """Per-(seed, layer, H, D) device sign tables, like the reference's signs_cache
    (hadamard_func.py:130-159)."""

    def __init__(self):
        self._lock = threading.Lock()
        self._cache: Dict[tuple, torch.Tensor] = {}

    def table(self, seed: int, layer_ids: Sequence[int], H: int, D: int, device) -> torch.Tensor:
        key = (seed, tuple(layer_ids), H, D, str(device))
        with self._lock:
            t = self._cache.get(key)
        if t is None:
            host = np.stack([rademacher_sign_bits(seed, l, H, D) for l in layer_ids])
            t = _upload(torch.from_numpy(host.view(np.int32)), device)
            with self._lock:
                self._cache[key] = t
        return t


SIGNS = _SignCache()


@dataclass
class Packet:
    """Device-resident result of compressing one request."""

    streams: List[torch.Tensor]          # uint8 per chunk: header + payload
    chunks: List[Tuple[int, int]]        # layer ranges [start, stop)
    kmeta: torch.Tensor                  # bf16 [L, 2, H, D]   (min, scale) by output position
    vmeta: torch.Tensor                  # bf16 [L, 2, G, B*S] (min, scale) by group
    profiles: List[LayerProfile]
    num_blocks: int
    block_size: int
    num_heads: int
    head_dim: int
    bits: int
    seed: int
    transform: bool
    layout: str
    layer_ids: List[int]
    axes: Tuple[str, str] = DEFAULT_AXES  # (axis_key, axis_value): how kmeta / vmeta are laid out

    @property
    def num_layers(self) -> int:
        return len(self.profiles)

    def layer_shape(self) -> Tuple[int, int, int, int, int]:
        return (2, self.num_blocks, self.block_size, self.num_heads, self.head_dim)

    def compressed_bytes(self) -> int:
        return sum(int(s.numel()) for s in self.streams)


AXES = ("channel", "token", "tensor")


def meta_shape(axis: str, H: int, D: int, G: int, ntok: int) -> Tuple[int, int]:
    """(rows, cols) of one layer's [min, scale] table of a part on `axis`: per channel
    by output position, per token by group, or one pair per group."""
    return {"channel": (H, D), "token": (G, ntok), "tensor": (G, 1)}[axis]


MAX_HEADS = 64        # kvmi_common.hpp kMaxHeads
MAX_ROW_SLOTS = 8192  # kvmi_common.hpp kMaxRowSlots: H * next_pow2(D)


def supported_geometry(num_heads: int, head_dim: int, bits: Optional[int] = None) -> bool:
    """The geometries the paged kernels take (kvmi_common.hpp check_geo): head_dim even
    in [2, 256] (split into power-of-two chunks when it is not one, hadamard_func.py:50-103,
    chunks below 16 channels included), 1..64 heads, heads * next_pow2(head_dim) <= 8192,
    and with a symbol width: whole-byte packed rows (head_dim * bits a multiple of 8)."""
    if type(num_heads) is not int or type(head_dim) is not int:
        return False
    if not 1 <= num_heads <= MAX_HEADS or not 2 <= head_dim <= 256 or head_dim % 2:
        return False
    if bits is not None and (head_dim * bits) % 8:
        return False
    return num_heads * (1 << (head_dim - 1).bit_length()) <= MAX_ROW_SLOTS


def check_geometry(num_heads: int, head_dim: int, bits: Optional[int] = None) -> None:
    if not supported_geometry(num_heads, head_dim, bits):
        raise ValueError(f"unsupported geometry: {num_heads} heads of head_dim {head_dim}"
                         + (f" at {bits} bits" if bits is not None else "")
                         + f" (head_dim even in [2, 256], 1..{MAX_HEADS} heads, heads * next_pow2(head_dim) <= "
                         f"{MAX_ROW_SLOTS}, head_dim * bits a multiple of 8)")


class FusedKVCodec:
    """Fused compress / decompress of paged KV for one worker's geometry.

    Parameters mirror the reference's configuration keys:
      bits       codec_config.bitpack_bits (bitpack_codec.py:87-91)
      seed       transformer_config.seed (kvserve_transformer.py:22)
      transform  "transformer" in the pipeline
      layout     KVSERVE_CODEC_LAYOUT permuted|native (compression_manager.py:136-140)
    """

    def __init__(self, num_heads: int, head_dim: int, block_size: int, bits: int = 4,
                 seed: int = DEFAULT_SEED, transform: bool = True, layout: str = "permuted",
                 header: bool = True, fwht: Optional[str] = None, compress_path: Optional[str] = None,
                 axes: Tuple[str, str] = DEFAULT_AXES):
        if type(bits) is not int or not 1 <= bits <= 8:
            raise ValueError("bitpack_bits must be an integer in [1, 8]")
        check_geometry(num_heads, head_dim, bits)
        if layout not in ("permuted", "native"):
            raise ValueError("layout must be 'permuted' or 'native'")
        if not header and bits != 8:
            raise ValueError("a stream without header carries raw 8-bit symbols")
        axes = tuple(axes)
        if len(axes) != 2 or any(a not in AXES for a in axes):
            raise ValueError("axes must be (axis_key, axis_value), each 'channel', 'token' or 'tensor'")
        self.axes = axes
        self.H, self.D, self.S, self.bits = num_heads, head_dim, block_size, bits
        self.seed, self.transform, self.layout, self.header = int(seed), transform, layout, header
        # Hadamard on MFMA (default), or forced onto the register FWHT kernels:
        # "valu" the quad-per-row kernels, "rows" the generic row kernels
        # (KVSERVE_AMD_FWHT=valu|rows)
        self.fwht = (fwht or os.environ.get("KVSERVE_AMD_FWHT", "mfma")).strip().lower()
        if self.fwht not in ("mfma", "valu", "rows"):
            raise ValueError("fwht must be 'mfma', 'valu' or 'rows'")
        # compress: "two_pass" (the default: kvmi_kstats_paged + kvmi_encode_paged, K read
        # twice; the faster on MI355X for short and long requests alike) or "one_pass"
        # (kvmi_compress_paged: every K value read from HBM once where the jobs fit the
        # one-pass kernel); KVSERVE_AMD_COMPRESS overrides the default
        self.compress_path = (compress_path or os.environ.get("KVSERVE_AMD_COMPRESS", "two_pass")).strip().lower()
        if self.compress_path not in ("one_pass", "two_pass"):
            raise ValueError("compress_path must be 'one_pass' or 'two_pass'")
        self._lib = _lib.load()
        self._prof_cache: Dict[tuple, torch.Tensor] = {}
        self._prof_valid: set = set()
        self._pools_ok: Dict[tuple, tuple] = {}
        self._stage_ring: List[tuple] = [(None, None)] * 4  # pinned upload buffers and their last copy's event
        self._stage_next = 0
        self._stage_last = 0

    # ---------------------------------------------------------------- helpers
    def _flags(self, max_level: int) -> int:
        f = 0
        if not self.transform:
            f |= _lib.F_NO_TRANSFORM
        if self.layout == "native":
            f |= _lib.F_NATIVE_LAYOUT
        if not self.header:
            f |= _lib.F_NO_HEADER
        if self.fwht == "valu":
            f |= _lib.F_VALU_FWHT
        elif self.fwht == "rows":
            f |= _lib.F_ROW_FWHT
        if max_level > 128:
            f |= _lib.F_CLAMP_LEVELS
        f |= {"channel": 0, "token": _lib.F_K_TOKEN, "tensor": _lib.F_K_TENSOR}[self.axes[0]]
        f |= {"token": 0, "channel": _lib.F_V_CHANNEL, "tensor": _lib.F_V_TENSOR}[self.axes[1]]
        return f

    def _groups_of(self, p: LayerProfile) -> int:
        """Statistic groups the metadata of profile p needs: V's groups, and K's when K
        shares statistics over groups (token / tensor axis)."""
        n = p.num_v_groups()
        if self.axes[0] != "channel":
            n = max(n, max(p.k_groups()) + 1)
        return n

    def _geometry(self, groups: int, max_level: int) -> _lib.Geometry:
        g = _lib.Geometry()
        g.block_size, g.num_heads, g.head_dim, g.bits = self.S, self.H, self.D, self.bits
        g.flags, g.max_groups = self._flags(max_level), groups
        return g

    def _kstats_scratch(self, L: int, device) -> torch.Tensor:
        """uint32 keys [L, 2, H, D] = {0xFFFFFFFF, 0} ([L, 2 parts, 2, H, D] when V takes
        a statistics pass too).  The kernels leave them initialised, so a plan reuses
        its own set on every run."""
        parts = 2 if self.axes[1] != "token" else 1
        keys = torch.empty((L, parts, 2, self.H, self.D), dtype=torch.int32, device=device)
        keys[:, :, 0].fill_(-1)
        keys[:, :, 1].zero_()
        return keys

    def _check_pools(self, pools: Sequence[torch.Tensor]) -> torch.device:
        """Device of the per-layer caches after checking dtype, shape, layout and
        placement; the caches of a deployment are the same tensors on every request,
        so a passing set is remembered by identity and address."""
        hit = self._pool_entry(pools)
        if hit[1] is None:
            self._pools_ok[hit[4]] = hit = hit[:1] + (self._check_pools_once(pools),) + hit[2:]
        return hit[1]

    def _pool_entry(self, pools: Sequence[torch.Tensor]) -> tuple:
        """(pools, device once checked or None, base addresses, elements per part, key)
        of a set of caches, remembered by identity and address."""
        key = tuple((id(p), p.data_ptr()) for p in pools)
        hit = self._pools_ok.get(key)
        if hit is not None and all(a is b for a, b in zip(hit[0], pools)):
            return hit
        if len(self._pools_ok) > 16:
            self._pools_ok.clear()
        hit = (tuple(pools), None, np.array([k[1] for k in key], np.int64),
               np.array([p.shape[1] * self.S * self.H * self.D for p in pools], np.int64), key)
        self._pools_ok[key] = hit
        return hit

    def _check_pools_once(self, pools: Sequence[torch.Tensor]) -> torch.device:
        if not pools:
            raise ValueError("at least one layer is required")
        dev = pools[0].device
        for p in pools:
            if p.dtype != torch.bfloat16:
                raise TypeError("KV caches must be bfloat16")
            if p.dim() != 5 or p.shape[0] != 2 or tuple(p.shape[2:]) != (self.S, self.H, self.D):
                raise ValueError(f"KV cache must be [2, num_blocks, {self.S}, {self.H}, {self.D}], got {tuple(p.shape)}")
            if not p.is_contiguous():
                raise ValueError("KV caches must be contiguous")
            if p.device != dev or p.device.type != "cuda":
                raise ValueError("KV caches must live on one GPU")
        return dev

    def _block_table(self, block_ids, device, pool_blocks: int):
        """The block table: a host int32 array, every id checked against the cache size
        here and uploaded with the plan's job table; or, for a device tensor, the int32
        device tensor, checked by the plan's first launch (kvmi_check_block_ids: a bad
        id sets the error the plan reports, zeroes every job's block count and so leaves
        the caches untouched), so that building a plan does not synchronize."""
        if isinstance(block_ids, torch.Tensor) and block_ids.is_cuda:
            if block_ids.dim() != 1:
                raise ValueError("block_ids must be 1-D")
            # the plan's own copy: the first run checks it once, and a caller that
            # rewrites its table in place later cannot slip unchecked ids under the plan
            return block_ids.to(device=device, dtype=torch.int32, copy=True).contiguous()
        ids = np.asarray(block_ids.numpy() if isinstance(block_ids, torch.Tensor) else block_ids, dtype=np.int64)
        if ids.ndim != 1:
            raise ValueError("block_ids must be 1-D")
        if ids.size and (int(ids.min()) < 0 or int(ids.max()) >= pool_blocks):
            raise IndexError("block id outside the KV cache")
        return ids.astype(np.int32)

    def _jobs(self, pools, ids, streams, chunks, kmeta, vmeta, signs, prof_dev, keys, B) -> torch.Tensor:
        """The kvmi_layer_job table: one row per layer, built with array arithmetic
        (per-layer pointers are base + l * layer stride of each table).  `ids` is the
        device block table, or a host int32 array: it is then uploaded in the same copy
        as the table (returned as the table's `block_ids` attribute)."""
        dev = pools[0].device
        L = len(pools)
        jb = L * _lib.JOB_INT64S * 8
        host_ids = None
        if isinstance(ids, torch.Tensor):
            up = torch.empty(jb, dtype=torch.uint8, device=dev)
        else:
            up = torch.empty(jb + 4 * max(1, ids.size), dtype=torch.uint8, device=dev)
            host_ids = ids
            ids = up[jb:jb + 4 * ids.size].view(torch.int32)
        rows = self._job_rows(pools, ids, streams, chunks, kmeta, vmeta, signs, prof_dev, keys, B)
        stage = self._staging(up.numel())
        host = stage.numpy()
        host[:rows.nbytes] = rows.view(np.uint8).reshape(-1)
        if host_ids is not None:
            host[rows.nbytes:rows.nbytes + host_ids.nbytes] = host_ids.view(np.uint8)
        up.copy_(stage, non_blocking=True)
        self._staged(dev)
        table = up[:rows.nbytes].view(torch.int64).view(rows.shape)
        table.block_ids = ids
        return table

    def _job_rows(self, pools, ids, streams, chunks, kmeta, vmeta, signs, prof_dev, keys, B) -> np.ndarray:
        L = len(pools)
        H, D, S = self.H, self.D, self.S
        per_layer = 2 * H * B * S * D
        lay = np.arange(L, dtype=np.int64)
        start = np.empty(L, np.int64)
        stop = np.empty(L, np.int64)
        stream = np.empty(L, np.int64)
        for (s, e), st in zip(chunks, streams):
            start[s:e], stop[s:e], stream[s:e] = s, e, _ptr(st)

        def strided(t):  # address of t[l] for every l (t contiguous along its first axis)
            return _ptr(t) + lay * (t.stride(0) * t.element_size()) if t is not None else np.zeros(L, np.int64)

        _, _, pool_ptrs, part_elems, _ = self._pool_entry(pools)
        rows = np.zeros((L, _lib.JOB_INT64S), dtype=np.int64)
        rows[:, 0] = pool_ptrs
        rows[:, 1] = _ptr(ids)
        rows[:, 2] = stream
        rows[:, 3] = strided(kmeta)
        rows[:, 4] = strided(vmeta)
        rows[:, 5] = strided(signs)
        rows[:, 6] = strided(prof_dev)
        rows[:, 7] = strided(keys)
        rows[:, 8] = part_elems // (S * H * D)  # pool blocks P of each layer
        rows[:, 9] = part_elems
        rows[:, 10] = (lay - start) * per_layer
        rows[:, 11] = (stop - start) * per_layer
        rows[:, 12] = B | ((lay == start).astype(np.int64) << 32)
        return rows

    def _staging(self, nbytes: int) -> torch.Tensor:
        """A pinned host buffer of `nbytes` for an asynchronous upload: the next slot of
        a small ring, waited on if its previous copy has not finished."""
        i = self._stage_next
        self._stage_next = (i + 1) % len(self._stage_ring)
        buf, ev = self._stage_ring[i]
        if ev is not None:
            ev.synchronize()
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, pin_memory=True)
        self._stage_ring[i] = (buf, None)
        self._stage_last = i
        return buf[:nbytes]

    def _staged(self, device) -> None:
        """Record the end of the upload (on `device`'s current stream) from the staging
        slot just filled."""
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(device))
        buf, _ = self._stage_ring[self._stage_last]
        self._stage_ring[self._stage_last] = (buf, ev)

    @staticmethod
    def _profile_key(profiles: Sequence[LayerProfile]) -> tuple:
        """The content of the profiles that validation and the device table depend on
        (a snapshot: a profile edited in place gets a new key)."""
        return tuple((tuple(p.k_order), tuple(p.k_levels), tuple(p.v_order), tuple(p.v_levels),
                      tuple(p.v_group), None if p.k_group is None else tuple(p.k_group)) for p in profiles)

    def _validate_profiles(self, profiles: Sequence[LayerProfile], key: tuple) -> None:
        """LayerProfile.validate on every profile, once per distinct content."""
        if key in self._prof_valid:
            return
        for p in profiles:
            p.validate(self.H, k_groups=self.axes[0] != "channel")
        if len(self._prof_valid) > 64:
            self._prof_valid.clear()
        self._prof_valid.add(key)

    def _profile_table(self, profiles: Sequence[LayerProfile], device, key: Optional[tuple] = None) -> torch.Tensor:
        """uint8 [L, 2, 3, H] device copy of the profiles, cached by their content (a
        caller that keeps its profile list, as the compression manager does, uploads it
        once)."""
        ck = (self._profile_key(profiles) if key is None else key, str(device))
        t = self._prof_cache.get(ck)
        if t is not None:
            return t
        t = _upload(torch.from_numpy(np.stack([p.to_array() for p in profiles])), device)
        if len(self._prof_cache) > 64:
            self._prof_cache.clear()
        self._prof_cache[ck] = t
        return t

    # ---------------------------------------------------------------- plans
    def plan_compress(self, pools: Sequence[torch.Tensor], block_ids, profiles: Sequence[LayerProfile],
                      layer_ids: Optional[Sequence[int]] = None, chunk_layers: Optional[int] = None,
                      groups: Optional[int] = None) -> "Plan":
        """Allocate the outputs and device descriptors for compressing blocks
        `block_ids` of every layer cache in `pools` (one tensor [2, P, S, H, D] per
        layer, vLLM FlashAttention NHD layout).  `run` then enqueues the kernels.

        layer_ids: the reference's layer index of each pool (sign seeds); by default
        0..L-1, the position in the connector's sorted layer list.
        chunk_layers: layers per stream; default = the reference's rule (one stream,
        or 8-layer chunks above 500 MiB); 0 = one stream.
        groups: V statistic groups the V metadata is laid out for (default: the most any
        layer of this request uses); plans batched together share one value."""
        dev = self._check_pools(pools)
        L = len(pools)
        if len(profiles) != L:
            raise ValueError("one profile per layer is required")
        self._validate_profiles(profiles, self._profile_key(profiles))
        layer_ids = list(range(L)) if layer_ids is None else [int(x) for x in layer_ids]
        ids = self._block_table(block_ids, dev, min(p.shape[1] for p in pools))
        B = int(ids.numel()) if isinstance(ids, torch.Tensor) else int(ids.size)
        H, D, S = self.H, self.D, self.S
        raw = L * 2 * B * S * H * D * 2
        if chunk_layers is None:
            chunks = chunk_ranges(L, raw)
        elif chunk_layers == 0:
            chunks = [(0, L)]
        else:
            chunks = [(s, min(s + chunk_layers, L)) for s in range(0, L, chunk_layers)]
        G = max(self._groups_of(p) for p in profiles)
        if groups is not None:
            if not G <= int(groups) <= H:
                raise ValueError("groups must cover every layer's statistic groups and be <= num_heads")
            G = int(groups)
        hdr = 16 if self.header else 0
        streams = []
        for s, e in chunks:
            n = (e - s) * 2 * H * B * S * D
            streams.append(torch.empty(hdr + (n * self.bits + 7) // 8, dtype=torch.uint8, device=dev))
        # both metadata tables live in one allocation: the reference's per-section
        # dicts are views of it, and the wire bundle ships it without a copy
        kshape = meta_shape(self.axes[0], H, D, G, B * S)
        vshape = meta_shape(self.axes[1], H, D, G, B * S)
        kn, vn = L * 2 * kshape[0] * kshape[1], L * 2 * vshape[0] * vshape[1]
        meta_buf = torch.empty(kn + vn, dtype=torch.bfloat16, device=dev)
        kmeta = meta_buf[:kn].view(L, 2, *kshape)
        vmeta = meta_buf[kn:].view(L, 2, *vshape)
        packet = Packet(streams, chunks, kmeta, vmeta, list(profiles), B, S, H, D, self.bits, self.seed,
                        self.transform, self.layout, layer_ids, self.axes)
        if B == 0 and self.header:
            for st in streams:
                st.copy_(_upload(torch.from_numpy(_header_bytes(self.bits, 0)), dev))
        return Plan(self, "compress", list(pools), ids, packet)

    def plan_decompress(self, packet: Packet, pools: Sequence[torch.Tensor], block_ids) -> "Plan":
        """Descriptors for writing `packet` into `pools` at `block_ids` (only the
        first packet.num_blocks ids are used, kv_utils.py:100-106)."""
        dev = self._check_pools(pools)
        if len(pools) != packet.num_layers:
            raise ValueError("one KV cache per compressed layer is required")
        if (packet.bits, packet.num_heads, packet.head_dim, packet.block_size) != (self.bits, self.H, self.D, self.S):
            raise ValueError("packet geometry does not match this codec")
        if (packet.seed, packet.transform, packet.layout) != (self.seed, self.transform, self.layout):
            raise ValueError("packet transform / layout does not match this codec")
        if tuple(packet.axes) != self.axes:
            raise ValueError("packet quantization axes do not match this codec")
        G = packet.vmeta.shape[2] if self.axes[1] != "channel" else (
            packet.kmeta.shape[2] if self.axes[0] != "channel" else 1)
        for name, t, axis in (("kmeta", packet.kmeta, self.axes[0]), ("vmeta", packet.vmeta, self.axes[1])):
            want = (packet.num_layers, 2) + meta_shape(axis, self.H, self.D, G, packet.num_blocks * self.S)
            if tuple(t.shape) != want:
                raise ValueError(f"{name} must be {list(want)} for axis {axis!r}, got {list(t.shape)}")
        ids = self._block_table(block_ids, dev, min(p.shape[1] for p in pools))
        if (ids.numel() if isinstance(ids, torch.Tensor) else ids.size) < packet.num_blocks:
            raise ValueError("fewer block ids than compressed blocks")
        ids = ids[: packet.num_blocks]
        ids = ids.contiguous() if isinstance(ids, torch.Tensor) else np.ascontiguousarray(ids)
        hdr = 16 if self.header else 0
        for (s, e), st in zip(packet.chunks, packet.streams):
            n = (e - s) * 2 * self.H * packet.num_blocks * self.S * self.D
            if st.dtype != torch.uint8 or st.dim() != 1:
                raise TypeError("packed streams are 1-D uint8 tensors")
            if st.numel() != hdr + (n * self.bits + 7) // 8:
                raise ValueError("BitPackCodec payload length does not match shape and bit width")
            if st.device != dev:
                raise ValueError("BitPackCodec decodes on the payload's CUDA device")
        # the kernels read streams with 16-byte loads: a view at an unaligned offset is
        # decoded from an aligned copy
        if any(st.data_ptr() % 16 for st in packet.streams):
            packet = dataclasses.replace(
                packet, streams=[st.clone() if st.data_ptr() % 16 else st for st in packet.streams])
        return Plan(self, "decompress", list(pools), ids, packet)

    # ---------------------------------------------------------------- one-shot API
    def compress(self, pools: Sequence[torch.Tensor], block_ids, profiles: Sequence[LayerProfile],
                 layer_ids: Optional[Sequence[int]] = None, chunk_layers: Optional[int] = None) -> Packet:
        plan = self.plan_compress(pools, block_ids, profiles, layer_ids, chunk_layers)
        plan.run()
        return plan.packet

    def decompress(self, packet: Packet, pools: Sequence[torch.Tensor], block_ids) -> None:
        self.plan_decompress(packet, pools, block_ids).run()

    # ---------------------------------------------------------------- batches
    def plan_compress_batch(self, requests: Sequence[tuple], chunk_layers: Optional[int] = None) -> "BatchPlan":
        """One plan for several requests: `requests` holds (pools, block_ids, profiles)
        or (pools, block_ids, profiles, layer_ids) tuples, each compressed into its own
        packet exactly as plan_compress would, with one launch per kernel for all of
        them (requests may differ in length and profile)."""
        reqs = [tuple(r) + (None,) * (4 - len(r)) for r in requests]
        if not reqs:
            raise ValueError("a batch needs at least one request")
        G = max(p.num_v_groups() for r in reqs for p in r[2])
        return BatchPlan([self.plan_compress(pools, ids, prof, lids, chunk_layers, groups=G)
                          for pools, ids, prof, lids in reqs])

    def plan_decompress_batch(self, items: Sequence[tuple]) -> "BatchPlan":
        """One plan writing several packets back: `items` holds (packet, pools,
        block_ids) tuples.  The packets must share their V metadata layout (as the
        packets of one plan_compress_batch do)."""
        return BatchPlan([self.plan_decompress(pk, pools, ids) for pk, pools, ids in items])


class Plan:
    """Device descriptors of one compress or decompress of one request.  `run()`
    enqueues the kernels on the current stream (two launches to compress, one to
    decompress) and can be repeated; the outputs are overwritten in place."""

    def __init__(self, codec: FusedKVCodec, kind: str, pools, ids: torch.Tensor, packet: Packet):
        self.codec, self.kind, self.pools, self.ids, self.packet = codec, kind, pools, ids, packet
        dev = pools[0].device
        self.device = dev
        L, B = len(pools), packet.num_blocks
        self.num_jobs, self.max_blocks = L, B
        self.signs = None
        if codec.transform:
            self.signs = SIGNS.table(codec.seed, packet.layer_ids, codec.H, codec.D, dev)
        self.prof = codec._profile_table(packet.profiles, dev)
        self.keys = codec._kstats_scratch(L, dev)
        self.jobs = codec._jobs(pools, ids, packet.streams, packet.chunks, packet.kmeta, packet.vmeta,
                                self.signs, self.prof, self.keys, B)
        # a device block table is checked by the first launch of the plan's first run
        # (the table is the plan's, as a host table would be checked once at build)
        self.check_ids, self._ids_checked = isinstance(ids, torch.Tensor), False
        if not self.check_ids:
            self.ids = self.jobs.block_ids  # uploaded with the job table
        self.err = torch.zeros(1, dtype=torch.int32, device=dev)
        max_level = max(max(max(p.k_levels), max(p.v_levels)) for p in packet.profiles)
        self.geo = codec._geometry(packet_groups(packet), max_level)
        packet.__dict__["_err"] = self.err
        self.job_blocks = np.full(L, B, dtype=np.int32)
        self._init_workspace()

    def _init_workspace(self) -> None:
        """Schedule and workspace of kvmi_compress_paged, built once per plan: the host
        schedule image (from every job's block count) and a device workspace holding a
        copy of it followed by zeroed barrier flags, keys and epoch.  No schedule (the
        one-pass kernel does not take these jobs): the plan runs the two passes."""
        self.schedule, self.workspace = None, None
        if self.kind != "compress" or self.codec.compress_path == "two_pass" or self.max_blocks == 0:
            return
        lib, geo = self.codec._lib, ctypes.byref(self.geo)
        nb = np.ascontiguousarray(self.job_blocks, dtype=np.int32)
        n = int(lib.kvmi_compress_schedule(geo, nb.ctypes.data, self.num_jobs, None, 0))
        if n < 0:
            _lib.check(n, "kvmi_compress_schedule")
        if n == 0:
            return
        img = np.zeros(n, dtype=np.uint8)
        _lib.check(min(0, int(lib.kvmi_compress_schedule(geo, nb.ctypes.data, self.num_jobs, img.ctypes.data, n))),
                   "kvmi_compress_schedule")
        total = int(lib.kvmi_compress_workspace_bytes(img.ctypes.data))
        ws = torch.zeros(total, dtype=torch.uint8, device=self.device)
        stage = self.codec._staging(n)
        stage.numpy()[:] = img
        ws[:n].copy_(stage, non_blocking=True)
        self.codec._staged(self.device)
        self.schedule, self.workspace = img, ws

    def launches(self) -> List[str]:
        """Names of the C entry points one run() enqueues, in order."""
        if self.max_blocks == 0:
            return []
        first = ["kvmi_check_block_ids"] if self.check_ids and not self._ids_checked else []
        if self.kind == "compress":
            if self.workspace is not None:
                return first + ["kvmi_compress_paged"]
            return first + ["kvmi_kstats_paged", "kvmi_encode_paged"]
        return first + ["kvmi_decode_paged"]

    def launch(self, name: str) -> None:
        """Enqueue one of launches() on the current stream."""
        fn = getattr(self.codec._lib, name)
        with torch.cuda.device(self.device):
            if name == "kvmi_check_block_ids":
                if not self._ids_checked:  # once per plan
                    _lib.check(fn(_ptr(self.jobs), self.num_jobs, _ptr(self.err), _stream_handle()), name)
                    self._ids_checked = True
                return
            if name == "kvmi_compress_paged":
                _lib.check(fn(ctypes.byref(self.geo), _ptr(self.jobs), self.num_jobs, self.max_blocks,
                              self.schedule.ctypes.data, _ptr(self.workspace), _ptr(self.err), _stream_handle()),
                           name)
                return
            _lib.check(fn(ctypes.byref(self.geo), _ptr(self.jobs), self.num_jobs, self.max_blocks, _ptr(self.err),
                          _stream_handle()), name)

    def run(self) -> None:
        for name in self.launches():
            self.launch(name)

    def error_code(self) -> int:
        """Synchronizes the stream and returns the sticky device error word."""
        return int(self.err.item())

    def check_errors(self) -> None:
        raise_device_error(self.error_code())


class BatchPlan:
    """Plans of one codec and direction enqueued together: their job tables are
    concatenated, so each C entry point is launched once for every layer of every
    request (each job keeps its own pools, block table, stream, metadata and scratch).
    All packets of the batch report device errors through one shared error word."""

    def __init__(self, plans: Sequence[Plan]):
        plans = list(plans)
        if not plans:
            raise ValueError("a batch needs at least one plan")
        p0 = plans[0]
        for p in plans[1:]:
            if p.codec is not p0.codec or p.kind != p0.kind or p.device != p0.device:
                raise ValueError("batched plans must share codec, direction and device")
            if p.geo.max_groups != p0.geo.max_groups:
                raise ValueError("batched packets must share their V metadata layout (groups)")
        self.plans, self.codec, self.kind, self.device = plans, p0.codec, p0.kind, p0.device
        self.packets = [p.packet for p in plans]
        self.num_jobs = sum(p.num_jobs for p in plans)
        self.max_blocks = max(p.max_blocks for p in plans)
        self.jobs = torch.cat([p.jobs for p in plans])
        self.check_ids, self._ids_checked = any(p.check_ids for p in plans), False
        max_level = max(max(max(pr.k_levels), max(pr.v_levels)) for p in plans for pr in p.packet.profiles)
        self.geo = p0.codec._geometry(p0.geo.max_groups, max_level)
        self.err = torch.zeros(1, dtype=torch.int32, device=self.device)
        for pk in self.packets:
            pk.__dict__["_err"] = self.err
        self.job_blocks = np.concatenate([p.job_blocks for p in plans])
        self._init_workspace()

    _init_workspace = Plan._init_workspace
    launches = Plan.launches
    launch = Plan.launch
    run = Plan.run
    error_code = Plan.error_code
    check_errors = Plan.check_errors


def packet_groups(packet: Packet) -> int:
    """G of a packet's metadata layout: the group rows of a token- or tensor-axis table
    (1 when both parts are on the channel axis)."""
    for t, axis in ((packet.vmeta, packet.axes[1]), (packet.kmeta, packet.axes[0])):
        if axis != "channel":
            return int(t.shape[2])
    return 1


def raise_device_error(code: int) -> None:
    """Raise the reference's device-assert messages (bitpack_codec.py:32, :38, :60)."""
    if code & _lib.ERR_SYMBOL_RANGE:
        raise RuntimeError("symbol exceeds bitpack_bits")
    if code & _lib.ERR_BAD_HEADER:
        raise RuntimeError("invalid bitpack header or decode configuration")
    if code & _lib.ERR_CORRUPT:
        raise RuntimeError("corrupt entropy-coded stream")
    if code & _lib.ERR_BLOCK_ID:
        raise IndexError("block id outside the KV cache")
    if code & _lib.ERR_SYNC:
        raise RuntimeError("one-pass compress: a workgroup barrier timed out or met keys of another call")
    if code & _lib.ERR_SCHEDULE:
        raise RuntimeError("one-pass compress: a job has more blocks than its schedule")


def check_packet(packet: Packet, force: bool = False) -> None:
    """Synchronize on the packet's last run and raise on a device data error.
    Skipped while the stream is being captured into a graph, and (unless `force`)
    when KVSERVE_AMD_CHECK_ERRORS=0 keeps calls asynchronous."""
    err = packet.__dict__.get("_err")
    if err is None or torch.cuda.is_current_stream_capturing():
        return
    if not force and os.environ.get("KVSERVE_AMD_CHECK_ERRORS", "1") == "0":
        return
    raise_device_error(int(err.item()))


def _header_bytes(bits: int, n: int) -> np.ndarray:
    h = np.zeros(16, np.uint8)
    h[0:4] = np.frombuffer(np.uint32(0x0150424B).tobytes(), np.uint8)
    h[4] = bits
    h[8:16] = np.frombuffer(np.uint64(n).tobytes(), np.uint8)
    return h
