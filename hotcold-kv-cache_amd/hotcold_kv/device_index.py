"""Device search index of one layer's cold stores (hc_index_add / hc_index_search).

The host stores (controller._Ring, hc_cold.cpp) keep every evicted token's
pre-RoPE key, value and position.  The reference also searches there: a CPU
faiss.IndexFlatIP scan per (layer, batch row) (controller.py:223-232,
274-293).  A layer of the 32k x 16 workload holds 16 rows x 30 720 tokens x 8
KV heads of 128-float search vectors, 2 GB per search, which host threads
cannot scan within a retrieval window of a fast decode loop.  DeviceIndex
keeps the same vectors in HBM and ranks them on the GPU with the host store's
arithmetic, so the hits are the same logical indices.  The rows themselves are
then gathered from the host store (hc_cold_gather).

The index mirrors each store's ring: slots are assigned exactly as
ColdStore::next_slot does (consecutive from the size until full, then from the
oldest), so physical slots agree and a hit's logical index addresses the host
store's row.
"""

import numpy as np
import torch

from . import _native as N


class DeviceIndex:
    """Search vectors of B cold stores (one layer), capacity cap each, in HBM:
    vec [B][VH][capT/64][VD/4][64][4] fp32 (tiles of 64 slots, VD a
    multiple of 4), VH = 1 (head mean) or H (per KV head).  With unit vectors (normalize) and VD a
    multiple of 8 it also keeps them rounded to fp16 (vec16), and a search
    with a normalised query first scans that copy, then scores exactly only
    the slots the fp16 scores cannot rule out (pass16=False: exact scan
    only).  The hits are the same either way."""

    def __init__(self, B, H, D, VD, VH, cap, device, normalize=True, pass16=True, scratch=None):
        if VH not in (1, H):
            raise ValueError("DeviceIndex: VH must be 1 or H")
        if VD % 4:
            raise ValueError("DeviceIndex: the vector width must be a multiple of 4")
        self.B, self.H, self.D, self.VD, self.VH, self.cap = int(B), int(H), int(D), int(VD), int(VH), int(cap)
        self.normalize = bool(normalize)
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.capT = (self.cap + 63) // 64 * 64
        self.vec = torch.empty((self.B, self.VH, self.capT // 64, self.VD // 4, 64, 4), dtype=torch.float32,
                               device=self.device)
        self.vec16 = None
        if pass16 and self.normalize and self.VD % 8 == 0:
            self.vec16 = torch.empty((self.B, self.VH, self.capT // 64, self.VD // 8, 64, 8), dtype=torch.float16,
                                     device=self.device)
        # the searches' key scratch: B*VH*capT 8-byte and 4-byte keys.  Indexes
        # whose searches are ordered on one stream may share one (scratch_for)
        self.keys, self.keys32 = scratch if scratch is not None else self.scratch_for(self.B, self.VH, self.capT,
                                                                                      self.device)
        if self.keys.numel() < self.B * self.VH * self.capT or self.keys32.numel() < self.B * self.VH * self.capT:
            raise ValueError("DeviceIndex: the shared key scratch is too small")
        self.size = np.zeros(self.B, dtype=np.int64)
        self.head = np.zeros(self.B, dtype=np.int64)
        self._lib = N.lib()

    @staticmethod
    def scratch_for(B, VH, capT, device):
        """Key scratch for searches of B*VH planes of capT slots."""
        n = int(B) * int(VH) * int(capT)
        return (torch.empty((n,), dtype=torch.int64, device=device),
                torch.empty((n,), dtype=torch.int32, device=device))

    def nbytes(self):
        """Bytes of the vectors (fp32 and the fp16 copy), without the key scratch."""
        return self.vec.numel() * 4 + (0 if self.vec16 is None else self.vec16.numel() * 2)

    def _slots(self, idx):
        """Physical slots (B, te) int32 for the tokens of idx (B, te) (>= 0:
        stored), advancing the rings; only the last cap tokens of a row
        survive an add (hc_cold_add)."""
        B, te = idx.shape
        slot_of = np.full((B, te), -1, dtype=np.int32)
        for b in range(B):
            kept = np.nonzero(idx[b] >= 0)[0]
            if kept.size > self.cap:
                kept = kept[kept.size - self.cap:]
            n = int(kept.size)
            if n == 0:
                continue
            size, head = int(self.size[b]), int(self.head[b])
            start = size if size < self.cap else head
            slot_of[b, kept] = (start + np.arange(n, dtype=np.int64)) % self.cap
            if size + n <= self.cap:
                self.size[b] = size + n
            elif size < self.cap:
                self.size[b], self.head[b] = self.cap, (size + n - self.cap) % self.cap
            else:
                self.head[b] = (head + n) % self.cap
        return slot_of

    def add(self, kpre, idx, stream=None):
        """Vectors of tokens idx >= 0 of kpre (B,H,te,D) fp32 on the device
        (idx (B,te) int64 on the host: the same evicted_idx the host stores
        get); on the current stream."""
        if kpre.dtype != torch.float32 or kpre.dim() != 4 or kpre.shape[0] != self.B or kpre.shape[1] != self.H \
                or kpre.shape[3] != self.D or kpre.device != self.device or kpre.stride(3) != 1:
            raise RuntimeError("DeviceIndex.add: kpre must be (B,H,te,D) fp32 rows on the index's device")
        idx = np.asarray(idx)
        te = int(kpre.shape[2])
        if idx.shape != (self.B, te):
            raise RuntimeError("DeviceIndex.add: idx must be (B, te)")
        slot_of = torch.from_numpy(self._slots(idx)).to(self.device, non_blocking=False)
        ks = kpre.stride()
        st = stream if stream is not None else torch.cuda.current_stream(self.device).cuda_stream
        N.check(self._lib.hc_index_add(self.B, self.H, self.D, self.VH, self.VD, int(self.normalize),
                                       kpre.data_ptr(), ks[0], ks[1], ks[2], te, slot_of.data_ptr(),
                                       self.vec.data_ptr(), None if self.vec16 is None else self.vec16.data_ptr(),
                                       self.capT, st), "hc_index_add")
        self._slot_of = slot_of            # kept until the launch has run (the next add replaces it)

    def search(self, q, R, hits, normalize_q=True, stream=None, hits_host=None, wait_event=None, done_event=None,
               pass16=True):
        """Top-R logical indices per (row, head) for queries q (B,VH,q_dim)
        fp32 on the device, into hits (B,VH,R) int64 on the device (-1 past
        each row's size); on `stream` (default: the current stream), after
        wait_event if given.  hits_host (pinned, like hits): the kernel
        writes the hits there too; done_event is recorded behind it.
        pass16=False: the exact scan even where the fp16 pass applies."""
        if q.dtype != torch.float32 or q.dim() != 3 or q.shape[0] != self.B or q.shape[1] != self.VH \
                or q.stride(2) != 1 or q.device != self.device:
            raise RuntimeError("DeviceIndex.search: q must be (B,VH,q_dim) fp32 on the index's device")
        if hits.dtype != torch.int64 or tuple(hits.shape) != (self.B, self.VH, int(R)) or not hits.is_contiguous():
            raise RuntimeError("DeviceIndex.search: hits must be a contiguous (B,VH,R) int64 tensor")
        if hits_host is not None and (hits_host.dtype != torch.int64 or hits_host.shape != hits.shape
                                      or not hits_host.is_contiguous() or hits_host.is_cuda):
            raise RuntimeError("DeviceIndex.search: hits_host must be a contiguous host tensor like hits")
        st = stream if stream is not None else torch.cuda.current_stream(self.device).cuda_stream
        sizes = np.ascontiguousarray(self.size, dtype=np.int64)
        heads = np.ascontiguousarray(self.head, dtype=np.int64)
        qs = q.stride()
        v16 = self.vec16 if pass16 else None
        N.check(self._lib.hc_index_search(self.B, self.VH, self.VD, self.cap, q.data_ptr(), qs[0], qs[1],
                                          int(q.shape[2]), int(bool(normalize_q)), self.vec.data_ptr(),
                                          None if v16 is None else v16.data_ptr(), int(self.normalize), self.capT,
                                          sizes.ctypes.data, heads.ctypes.data, int(R), self.keys.data_ptr(),
                                          None if v16 is None else self.keys32.data_ptr(), hits.data_ptr(),
                                          None if hits_host is None else hits_host.data_ptr(),
                                          wait_event, done_event, st), "hc_index_search")
        return hits

    def vectors(self, b):
        """Row b's vectors as (VH, VD, capT), slot-indexed (a view over the tiles)."""
        return self.vec[b].permute(0, 2, 4, 1, 3).reshape(self.VH, self.VD, self.capT)

    def physical(self, b, logical):
        """Physical slot of logical index `logical` of row b."""
        if self.size[b] < self.cap:
            return logical
        return (self.head[b] + logical) % self.cap
