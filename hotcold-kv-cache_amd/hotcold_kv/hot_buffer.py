"""Fixed-capacity device storage of one layer's hot tier.

Layout (per layer): keys and values in one allocation [B][H][cap][2][D], so
a row's key and value are adjacent (exposed as two (B,H,cap,D) views of row
stride 2*D); optionally pre-RoPE keys [B][H][cap][D]; all in the cache
dtype; positions as [B][cap] int64.  Rows
0 .. held-1 are the held retrieved slot (written by the inject kernel), rows
held .. held+n-1 the resident hot tokens.  Appends write one row in place
(replacing the per-step torch.cat of cache.py:145-148 and
layer_state.py:99-100); compaction gathers into a second buffer and swaps,
so no row is read after it was overwritten.  Capacity grows geometrically
when an append would overflow.
"""

import torch

from . import ops


def kv_rows(prefix, rows, head_dim, dtype, device):
    """Key and value rows with each row's key and value adjacent in memory:
    one allocation [*prefix][rows][2][head_dim], returned as two
    (*prefix, rows, head_dim) views of row stride 2*head_dim, so decode reads
    each (batch, head) as one stream instead of two.  Timed against separate
    K and V tensors and two head-interleaved layouts, the 32-layer
    8k-context decode launch differs by less than 0.7 us (15.5-16.2 us for
    72 MB) and in no consistent order; the layout is kept for its one
    allocation per layer.  Every kernel that reads or writes hot rows takes
    row strides."""
    kv = torch.empty((*prefix, rows, 2, head_dim), dtype=dtype, device=device)
    return kv[..., 0, :], kv[..., 1, :]


class HotBuffer:
    def __init__(self, batch, heads, head_dim, dtype, device, capacity, held=0, with_pre=False, with_pos=False,
                 storage=None):
        """storage: optional (k, v) tensors (B,H,held+capacity,D) to use as the
        buffer's rows instead of allocating them (e.g. views of one allocation
        shared by many layers)."""
        self.B, self.H, self.D = int(batch), int(heads), int(head_dim)
        self.dtype, self.device = dtype, torch.device(device)
        self.held = int(held)
        self.with_pre, self.with_pos = with_pre, with_pos
        self.n = 0
        if storage is not None:
            if with_pre or with_pos or held:
                raise ValueError("HotBuffer: external storage holds K and V rows only")
            k, v = storage
            self.cap = int(k.shape[2])
            self.st = {"k": k, "v": v}
        else:
            self._alloc(max(1, int(capacity)))
        self._spare = None

    # -- storage --------------------------------------------------------------
    def _new_storage(self, cap):
        # Hot rows are written before any read (decode reads rows below
        # held + n only), so only the held slot -- attended masked until an
        # inject fills it, and a masked row still enters the P.V product with
        # weight 0 -- is zero-filled.
        shape = (self.B, self.H, self.held + cap, self.D)
        k, v = kv_rows((self.B, self.H), self.held + cap, self.D, self.dtype, self.device)
        st = {"k": k, "v": v}
        if self.with_pre:
            st["p"] = torch.empty(shape, dtype=self.dtype, device=self.device)
        if self.held:
            for name in ("k", "v", "p"):
                if name in st:
                    st[name][:, :, :self.held].zero_()
        if self.with_pos:
            st["pos"] = torch.zeros((self.B, self.held + cap), dtype=torch.int64, device=self.device)
        return st

    def _alloc(self, cap):
        self.cap = cap
        self.st = self._new_storage(cap)

    @property
    def capacity(self):
        return self.cap

    def ensure(self, rows):
        """Make room for `rows` hot rows, keeping the current contents."""
        if rows <= self.cap:
            return
        new_cap = max(rows, 2 * self.cap)
        old = self.st
        self.st = self._new_storage(new_cap)
        self.cap = new_cap
        self._spare = None
        total = self.held + self.n
        if total:
            ops.append_rows(0, old["k"][:, :, :total], self.st["k"], old["v"][:, :, :total], self.st["v"],
                            old["p"][:, :, :total] if self.with_pre else None,
                            self.st["p"] if self.with_pre else None,
                            pos_src=old["pos"][:, :total] if self.with_pos else None,
                            pos_dst=self.st["pos"] if self.with_pos else None)

    # -- views ------------------------------------------------------------------
    def _rows(self, name, start, stop):
        t = self.st[name]
        return t[:, start:stop] if name == "pos" else t[:, :, start:stop]

    @property
    def keys(self):
        return self._rows("k", self.held, self.held + self.n)

    @property
    def values(self):
        return self._rows("v", self.held, self.held + self.n)

    @property
    def pre_keys(self):
        return self._rows("p", self.held, self.held + self.n) if self.with_pre else None

    @property
    def positions(self):
        return self._rows("pos", self.held, self.held + self.n) if self.with_pos else None

    def attended(self, with_held):
        """(keys, values) of the rows decode attends: held slot + hot rows, or
        the hot rows only."""
        start = 0 if with_held else self.held
        return self._rows("k", start, self.held + self.n), self._rows("v", start, self.held + self.n)

    def held_storage(self):
        """Full-width k/v tensors whose rows 0..held-1 are the held slot."""
        return self.st["k"], self.st["v"]

    # -- mutation ----------------------------------------------------------------
    def append(self, k, v, pre=None, pos=None):
        """Append T tokens: k, v, pre (B,H,T,D) and pos (B,T) int64."""
        T = int(k.shape[2])
        self.ensure(self.n + T)
        row = self.held + self.n
        ops.append_rows(row, k, self.st["k"], v, self.st["v"],
                        pre if self.with_pre else None, self.st["p"] if self.with_pre else None,
                        pos_src=pos if self.with_pos else None, pos_dst=self.st["pos"] if self.with_pos else None)
        self.n += T

    def append_attend(self, q, k, v, scaling, pre=None, pos=None, keepdim=False):
        """Append one token (k, v, pre (B,H,1,D), pos (B,1)) and attend q over
        the hot rows plus the token, in one launch.  Returns (B,Hq,D), or
        (B,Hq,1,D) with keepdim."""
        n = self.n + 1
        if n > self.cap:
            self.ensure(n)
        out = ops.decode_append_rows(q, self.st, self.held, n, k, v, scaling, pre if self.with_pre else None,
                                     pos if self.with_pos else None, None, None, keepdim)
        self.n = n
        return out

    def set_from(self, k, v, pre=None, pos=None):
        """Replace the hot rows with the given tokens."""
        self.n = 0
        self.append(k, v, pre, pos)

    def spare(self):
        """The second storage (same capacity), which out-of-place compactions
        write into before adopt_spare makes it current."""
        if self._spare is None or self._spare["k"].shape[2] != self.held + self.cap:
            self._spare = self._new_storage(self.cap)
        return self._spare

    def spare_rows(self, name):
        """Hot rows (from row `held` on, full capacity) of the second storage."""
        return self.spare()[name][:, :, self.held:]

    def adopt_spare(self, n):
        """Make the second storage current with n hot rows (written there out
        of place); the held slot travels with the buffer."""
        dst = self.spare()
        if self.held:
            ops.append_rows(0, self.st["k"][:, :, :self.held], dst["k"], self.st["v"][:, :, :self.held], dst["v"])
        self._spare, self.st = self.st, dst
        self.n = int(n)

    def compact(self, keep):
        """Keep rows keep (B,H,n) per head or (B,n) shared, in that order."""
        n_keep = int(keep.shape[-1])
        dst = self.spare()
        pairs = [(self.keys, dst["k"]), (self.values, dst["v"])]
        if self.with_pre:
            pairs.append((self.pre_keys, dst["p"]))
        ops.gather_rows(keep, pairs, dst_row0=self.held,
                        pos_src=self.positions if self.with_pos else None,
                        pos_dst=dst["pos"] if self.with_pos else None)
        self.adopt_spare(n_keep)

    def gather_from(self, k, v, keep, pre=None, pos=None):
        """Fill the hot rows with rows keep of external tensors (B,H,S,D)."""
        n_keep = int(keep.shape[-1])
        self.ensure(n_keep)
        pairs = [(k, self.st["k"]), (v, self.st["v"])]
        if self.with_pre and pre is not None:
            pairs.append((pre, self.st["p"]))
        ops.gather_rows(keep, pairs, dst_row0=self.held,
                        pos_src=pos if (self.with_pos and pos is not None) else None,
                        pos_dst=self.st["pos"] if (self.with_pos and pos is not None) else None)
        self.n = n_keep
