"""On-disk fp16 archive of a layer's far-tier rows.

Same file format as the reference (samfurr/foveated_kv
src/foveated_kv/disk_archive.py:127-185): per layer two raw little-endian
fp16 files ``archive_k_layer{i}.bin`` / ``archive_v_layer{i}.bin`` of shape
(H_kv, S_arc, D), batch 0 only (the reference asserts B == 1), read back
through ``numpy.memmap``.  ``PromotionPipeline.register_archive`` takes the
two paths; the promoter copies the rows it needs into pinned host memory.
"""

from dataclasses import dataclass
from pathlib import Path
from typing import Optional, Union

import numpy as np
import torch


@dataclass
class DiskArchive:
    """disk_archive.py:27-124: memmapped (H_kv, S_arc, D) fp16 K and V rows
    plus the int32 position map ``idx`` (B, H_kv, S_arc), kept in memory."""

    path_k: str
    path_v: str
    mmap_k: np.memmap
    mmap_v: np.memmap
    idx: torch.Tensor
    H_kv: int
    S_arc: int
    D: int

    def promote(self, head: int, archive_local_idx: int):
        """Exact fp16 K, V of one archived token as (1, 1, 1, D) tensors."""
        k = torch.from_numpy(np.array(self.mmap_k[head, archive_local_idx, :]))
        v = torch.from_numpy(np.array(self.mmap_v[head, archive_local_idx, :]))
        return k.reshape(1, 1, 1, self.D), v.reshape(1, 1, 1, self.D)

    def promote_batch(self, head: int, archive_local_indices):
        """(1, 1, N, D) fp16 K, V for the listed archive-local indices."""
        n = len(archive_local_indices)
        if n == 0:
            z = torch.zeros((1, 1, 0, self.D), dtype=torch.float16)
            return z, z.clone()
        ix = np.asarray(archive_local_indices, dtype=np.int64)
        k = torch.from_numpy(np.array(self.mmap_k[head, ix, :]))
        v = torch.from_numpy(np.array(self.mmap_v[head, ix, :]))
        return k.reshape(1, 1, n, self.D), v.reshape(1, 1, n, self.D)

    def score_boundary_tokens(self, head: int, query: np.ndarray, token_indices) -> np.ndarray:
        """fp32 dot products of archived keys with ``query`` (D,)."""
        if len(token_indices) == 0:
            return np.array([], dtype=np.float32)
        k = self.mmap_k[head, np.asarray(token_indices, dtype=np.int64), :].astype(np.float32)
        return k @ np.asarray(query, dtype=np.float32)

    def memory_bytes_in_ram(self) -> int:
        return self.idx.numel() * self.idx.element_size()

    def disk_bytes(self) -> int:
        return self.H_kv * self.S_arc * self.D * 2 * 2

    def close(self):
        self.mmap_k = None
        self.mmap_v = None


def create_disk_archive(archive_k, archive_v, archive_idx, layer_idx: int,
                        archive_dir: Union[str, Path]) -> Optional[DiskArchive]:
    """disk_archive.py:127-185: write batch 0 of (B, H_kv, S_arc, D) archive
    rows as raw fp16 files; ``None`` when there is nothing to archive."""
    if archive_k.shape[0] != 1:
        raise ValueError(f"the on-disk archive holds one sequence (B=1), got B={archive_k.shape[0]}")
    _, H, S, D = archive_k.shape
    if S == 0:
        return None
    d = Path(archive_dir)
    d.mkdir(parents=True, exist_ok=True)
    path_k = str(d / f"archive_k_layer{layer_idx}.bin")
    path_v = str(d / f"archive_v_layer{layer_idx}.bin")
    archive_k[0].detach().to("cpu", torch.float16).contiguous().numpy().tofile(path_k)
    archive_v[0].detach().to("cpu", torch.float16).contiguous().numpy().tofile(path_v)
    mk = np.memmap(path_k, dtype=np.float16, mode="r", shape=(H, S, D))
    mv = np.memmap(path_v, dtype=np.float16, mode="r", shape=(H, S, D))
    return DiskArchive(path_k, path_v, mk, mv, archive_idx, H, S, D)


def offload_cache_to_disk(cache, archive_dir: Union[str, Path]) -> list:
    """disk_archive.py:188-222: move every layer's archive to disk and leave
    empty (1, H_kv, 0, D) placeholders in the layers; returns one
    ``DiskArchive`` (or None) per layer."""
    out = []
    for i, layer in enumerate(cache.layers):
        if layer is None:
            out.append(None)
            continue
        out.append(create_disk_archive(layer.archive_k, layer.archive_v, layer.archive_idx, i, archive_dir))
        H, D = layer.archive_k.shape[1], layer.archive_k.shape[3]
        dev = layer.archive_k.device
        layer.archive_k = torch.zeros((1, H, 0, D), dtype=torch.float16, device=dev)
        layer.archive_v = torch.zeros((1, H, 0, D), dtype=torch.float16, device=dev)
    return out
