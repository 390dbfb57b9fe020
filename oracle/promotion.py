"""CPU restatement of the reference's promotion pipeline -- TEST
INFRASTRUCTURE ONLY (imported by tests/ only).

drain():   csrc/promotion_pipeline.cpp:99-175 (GQA dedup, per-(layer, KV
           head) cooldown, position dedup, per-call budget, archive lookup).
           With spike_k > 1 (the benchmark's "up to 32 far tokens per head
           per step", an extension): flags[b, hq] is the number of spiking
           tokens of the query head and tokens (B, Hq, K) lists them in
           descending score order; the KV head's first flagged query head
           (GQA dedup) hands its tokens, in that order, through the same
           position dedup / archive lookup / budget, the budget checked
           before each token.  spike_k = 1 is the reference's drain.
commit():  csrc/promotion_pipeline.cpp:192-241 (headroom check against
           N_near_alloc, copy the fp16 K/V row into slot near_valid[h],
           near_valid[h] += 1).

Parity of this restatement is pinned by the known answers in
tests/test_promotion.py (hand-worked flag streams for each rule) and by the
reference's own archive test (tests/test_disk_archive.py:25-49: a promoted
row is the bit-exact original row).
"""

import numpy as np

STATS = ("spikes_detected", "spikes_queued", "spikes_deduplicated", "spikes_cooled_down",
         "promotions_completed", "promotions_headroom_full")


class Pipeline:
    def __init__(self, n_layers, cooldown_steps=5, max_per_drain=8, spike_k=1):
        self.n_layers = n_layers
        self.cooldown = cooldown_steps
        self.max_per_drain = max_per_drain
        self.spike_k = spike_k
        self.archives = {}  # layer -> (k, v, pos_to_local list of dicts)
        self.promoted = set()
        self.last_step = {}
        self.queue = []
        self.stats = {s: 0 for s in STATS}

    def register_archive(self, layer, k, v, archive_idx):
        """k, v: (B_arc, H_kv, S_arc, D) fp16; archive_idx (H_kv, S_arc)."""
        maps = [{int(p): i for i, p in enumerate(archive_idx[h])} for h in range(archive_idx.shape[0])]
        self.archives[layer] = (k, v, maps)

    def drain(self, layer, flags, tokens, far_idx, step):
        if layer < 0 or layer >= self.n_layers or layer not in self.archives:
            return 0
        _, _, maps = self.archives[layer]
        B, Hq = flags.shape
        tokens = np.asarray(tokens).reshape(B, Hq, -1)
        Hkv, n_far = far_idx.shape[1], far_idx.shape[2]
        gqa = max(Hq // Hkv, 1)
        seen = [False] * Hkv
        queued = 0
        for b in range(B):
            if queued >= self.max_per_drain:
                break
            for hq in range(Hq):
                if queued >= self.max_per_drain:
                    break
                if flags[b, hq] == 0:
                    continue
                hkv = hq // gqa
                if hkv >= Hkv or seen[hkv]:
                    continue
                seen[hkv] = True
                self.stats["spikes_detected"] += 1
                key_cd = (layer, hkv)
                if key_cd in self.last_step and step - self.last_step[key_cd] < self.cooldown:
                    self.stats["spikes_cooled_down"] += 1
                    continue
                self.last_step[key_cd] = step
                n_tok = min(int(flags[b, hq]), self.spike_k) if self.spike_k > 1 else 1
                for j in range(n_tok):
                    if queued >= self.max_per_drain:
                        break
                    fl = int(tokens[b, hq, j])
                    if fl < 0 or fl >= n_far:
                        continue
                    pos = int(far_idx[b, hkv, fl])
                    key = (layer, hkv, pos)
                    if key in self.promoted:
                        self.stats["spikes_deduplicated"] += 1
                        continue
                    self.promoted.add(key)
                    if pos not in maps[hkv]:
                        continue
                    self.queue.append((layer, hkv, maps[hkv][pos], pos))
                    self.stats["spikes_queued"] += 1
                    queued += 1
        return queued

    def commit(self, near_k, near_v, near_valid, n_near_alloc):
        """Apply queued records to per-layer near tiers (dict layer -> arrays
        (B, H_kv, N_alloc, D)) and near_valid (dict layer -> (H_kv,))."""
        for layer, h, arc, _pos in self.queue:
            k, v, _ = self.archives[layer]
            cur = int(near_valid[layer][h])
            if cur >= n_near_alloc[layer]:
                self.stats["promotions_headroom_full"] += 1
                continue
            nb = k.shape[0]
            near_k[layer][:nb, h, cur] = k[:, h, arc]
            near_v[layer][:nb, h, cur] = v[:, h, arc]
            near_valid[layer][h] = cur + 1
            self.stats["promotions_completed"] += 1
        self.queue = []
