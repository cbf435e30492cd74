"""The calls M*'s KV-cache engine makes on the KV-cache classes, replayed in order.

``KVCacheEngine`` (``mstar/engine/kv_cache_engine.py``) builds one
``PagedAllocationManager`` per KV cache, keys it by ``KVCacheConfig.get_node_str()``,
reads its ``write_policy`` whenever it creates a ``BatchedCacheManager``, reads
``get_labels``/``get_state(...).get_pos_info()`` for every request of every
batch, writes the producer state back with ``get_per_label_seq_info``, sets the
policy for the whole worker and calls ``cleanup()`` at shutdown.  ``MiniEngine``
below makes those calls, with the same arguments and in the same order as the
cited lines, on this package's classes, so a test can show that the classes
swap in under the engine unchanged.  It holds only the manager-facing part of
the engine: no submodules, sampler, TP groups or CUDA-graph runner.
"""

from __future__ import annotations

import os
from dataclasses import dataclass

import torch

from mstar_amd.cache_manager import BatchedCacheManager, WorkspaceBufferManager
from mstar_amd.kv_store import (KVCacheConfig, PagedAllocationManager, StoreWritePolicy,
                                TransferEngineInfo)


class StubTransferEngine:
    """Single-node transport stand-in, as in the reference's integration tests
    (``test/integration/test_prefill_cuda_graph.py:76-97``): records
    registrations, has no async reader."""

    def __init__(self):
        self.registered: list[tuple[int, int]] = []

    def register_memory(self, ptr: int, nbytes: int) -> int:
        self.registered.append((ptr, nbytes))
        return 0

    def unregister_memory(self, ptr: int) -> int:
        return 0

    def get_async_reader(self, device):
        return None


class LocalTransferEngine(StubTransferEngine):
    """Same name as the reference's single-node transport
    (``mstar/communication/tensors.py:292-307``)."""


class MooncakeTransferEngine:
    """Same name as the reference's RDMA transport (``tensors.py:240``): an async
    reader exists, so page reads would cross nodes."""

    def get_async_reader(self, device):
        return object()


@dataclass
class KVManagement:
    """``kv_cache_engine.py:37-43``."""

    kv_cache_config: KVCacheConfig
    kv_cache: torch.Tensor | None
    alloc_manager: PagedAllocationManager
    buffer_manager: WorkspaceBufferManager | None


class MiniEngine:
    def __init__(self, configs: list[KVCacheConfig], device: torch.device, transfer_engine_info: TransferEngineInfo,
                 kv_cache_type: torch.dtype = torch.bfloat16, workspace_mb: int | None = None):
        """``load_model``'s cache loop (``kv_cache_engine.py:107-163``), one TP rank."""
        self.device = device
        self.kv_management: dict[str, KVManagement] = {}
        for cfg in configs:
            cfg.shard(1)
            kv_cache = torch.zeros(cfg.num_layers, cfg.max_num_pages, 2, cfg.page_size, cfg.num_kv_heads,
                                   cfg.head_dim, dtype=kv_cache_type, device=device).contiguous()
            mb = workspace_mb if workspace_mb is not None else int(os.environ.get("MSTAR_WORKSPACE_BUFFER_MB", "512"))
            kv_mgmt = KVManagement(
                kv_cache_config=cfg,
                kv_cache=kv_cache,
                alloc_manager=PagedAllocationManager(
                    config=cfg,
                    kv_cache=kv_cache,
                    transfer_engine_info=transfer_engine_info,
                ),
                buffer_manager=WorkspaceBufferManager(mb * 1024 * 1024, device=device),
            )
            self.kv_management[cfg.get_node_str()] = kv_mgmt

    def create_cache_manager(self, key: str, request_ids: list[str]) -> BatchedCacheManager:
        """``_create_cache_manager`` (``kv_cache_engine.py:184-205``)."""
        cache_mgmt = self.kv_management[key]
        autowrite = (cache_mgmt.alloc_manager.write_policy == StoreWritePolicy.ALWAYS)
        return BatchedCacheManager(
            request_ids=request_ids,
            active_labels_per_request={rid: "main" for rid in request_ids},
            kv_cache=cache_mgmt.kv_cache,
            alloc_manager=cache_mgmt.alloc_manager,
            buffer_manager=cache_mgmt.buffer_manager,
            kv_cache_config=cache_mgmt.kv_cache_config,
            device=self.device,
            auto_write_store=autowrite,
            enable_nvtx=False,
        )

    def add_request(self, request_id: str, cache_labels: list[str] | None = None) -> None:
        """``kv_cache_engine.py:1037-1041``."""
        for m in self.kv_management.values():
            m.alloc_manager.add_request(request_id, cache_labels or ["main"])

    def pos_infos(self, key: str, request_ids: list[str]) -> dict:
        """The per-request position info ``prepare_batch`` hands to
        ``prepare_inputs`` (``kv_cache_engine.py:789-796``)."""
        cache_mgmt = self.kv_management[key]
        out = {}
        for rid in request_ids:
            labels = cache_mgmt.alloc_manager.get_labels(rid)
            out[rid] = {label: cache_mgmt.alloc_manager.get_state(rid, label).get_pos_info() for label in labels}
        return out

    def sync_retrieve(self, key: str, request_id: str, per_label_seq_info: dict) -> None:
        """``prepare_batch``'s retrieve loop (``kv_cache_engine.py:760-768``)."""
        cache_mgmt = self.kv_management[key]
        for label, seq_info in per_label_seq_info.items():
            cache_mgmt.alloc_manager.sync_retrieve(request_id, label, seq_info)

    def finalize(self, key: str, request_ids: list[str]) -> dict:
        """``finalize_batch``'s write-back (``kv_cache_engine.py:724-737``):
        the per-label producer state of every request."""
        cache_mgmt = self.kv_management[key]
        return {rid: cache_mgmt.alloc_manager.get_per_label_seq_info(rid) for rid in request_ids}

    def set_alloc_write_policy(self, policy: StoreWritePolicy) -> None:
        """``kv_cache_engine.py:1091-1093``."""
        for m in self.kv_management.values():
            m.alloc_manager.write_policy = policy

    def offload_candidates(self, key: str) -> list[tuple[str, int]]:
        """``kv_cache_engine.py:1095-1105``: reads ``request_states`` directly."""
        alloc = self.kv_management[key].alloc_manager
        out = []
        for rid, labels in alloc.request_states.items():
            total_pages = sum(len(s.page_indices) for s in labels.values())
            if total_pages > 0:
                out.append((rid, total_pages))
        return out

    def free_pages(self, key: str) -> int:
        """``_verify_tp_kv_symmetry`` (``kv_cache_engine.py:331``)."""
        return self.kv_management[key].alloc_manager.page_allocator.num_free

    def remove_request(self, request_id: str) -> None:
        """``kv_cache_engine.py:1049-1054``."""
        for m in self.kv_management.values():
            m.alloc_manager.remove_request(request_id)

    def shutdown(self) -> None:
        """``kv_cache_engine.py:1145-1150``."""
        for m in self.kv_management.values():
            m.kv_cache = None
            m.buffer_manager = None
            m.alloc_manager.cleanup()
