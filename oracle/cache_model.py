"""Restatement of the reference's VRAM expert cache and of the executor's admission
and byte accounting, as plain Python bookkeeping.

TEST INFRASTRUCTURE ONLY: tests/ use it as the checker for the library's cache
counters and MoE telemetry; nothing in the product imports it.

Follows crates/objeta-cuda/src/moe.rs:
  CudaExpertCache::{new,get,insert,touch,evict_lru,pin,insert_pinned,clear,reset_counters}
      moe.rs:91-226
  per-expert admission (oversized expert bypass / self-eviction risk) and the
  get -> miss -> copy -> insert sequence of execute_selected_moe_cuda
      moe.rs:458-583
  the same for the six split-FP4 tensors (load_tensor_to_device) moe.rs:753-814, 955-1100
  MoeTelemetry byte fields moe.rs:666-748, 1216-1270

Two deliberate differences, shared with the library: when only pinned entries are
left, `insert` stops evicting instead of looping forever (moe.rs:145-147 loops while
`order` is non-empty even when evict_lru finds nothing to evict); and re-inserting
a key with `insert_pinned` moves it to the most-recent end instead of leaving a
second copy of the key in `order` (moe.rs:200-208 pushes without removing).
"""
from __future__ import annotations

from dataclasses import dataclass, field

# ExpertTensorKind (moe.rs:37-54)
GATE, UP, DOWN = 0, 1, 2
GATE_WEIGHT, GATE_SCALE, UP_WEIGHT, UP_SCALE, DOWN_WEIGHT, DOWN_SCALE = 3, 4, 5, 6, 7, 8
SCALE_KINDS = {GATE_SCALE, UP_SCALE, DOWN_SCALE}
Q4_0, FP4 = 0, 3

COUNTERS = ("hit_count", "miss_count", "eviction_count", "cache_insert_attempt_count",
            "cache_insert_accept_count", "cache_insert_bypass_count", "oversized_tensor_bypass_count",
            "oversized_expert_bypass_count", "self_eviction_risk_count")


@dataclass
class CacheModel:
    """CudaExpertCache (moe.rs:70-226); keys are (layer, expert, kind, format)."""
    capacity_bytes: int
    resident_bytes: int = 0
    pinned_bytes: int = 0
    hit_count: int = 0
    miss_count: int = 0
    eviction_count: int = 0
    bypass_oversized_experts: bool = False
    cache_insert_attempt_count: int = 0
    cache_insert_accept_count: int = 0
    cache_insert_bypass_count: int = 0
    oversized_tensor_bypass_count: int = 0
    oversized_expert_bypass_count: int = 0
    self_eviction_risk_count: int = 0
    pinned: set = field(default_factory=set)
    sizes: dict = field(default_factory=dict)
    order: list = field(default_factory=list)

    def get(self, key) -> bool:  # moe.rs:113-122
        if key in self.sizes:
            self.hit_count += 1
            self.touch(key)
            return True
        self.miss_count += 1
        return False

    def insert(self, key, size: int) -> bool:  # moe.rs:124-158; True if cached
        self.cache_insert_attempt_count += 1
        if size > self.capacity_bytes:
            self.oversized_tensor_bypass_count += 1
            self.cache_insert_bypass_count += 1
            return False
        self.cache_insert_accept_count += 1
        if key in self.sizes:
            self.resident_bytes -= self.sizes.pop(key)
            if key in self.order:
                self.order.remove(key)
        while self.resident_bytes + size > self.capacity_bytes and self.order:
            if self.evict_lru() is None:
                break
        self.sizes[key] = size
        self.resident_bytes += size
        self.order.append(key)
        return True

    def touch(self, key) -> None:  # moe.rs:160-165
        if key in self.order:
            self.order.remove(key)
            self.order.append(key)

    def evict_lru(self):  # moe.rs:167-180
        for i, k in enumerate(self.order):
            if k not in self.pinned:
                del self.order[i]
                if k in self.sizes:
                    self.resident_bytes -= self.sizes.pop(k)
                    self.eviction_count += 1
                    return k
                return None
        return None

    def pin(self, key) -> None:  # moe.rs:182-190
        if key in self.sizes and key not in self.pinned:
            self.pinned.add(key)
            self.pinned_bytes += self.sizes[key]

    def insert_pinned(self, key, size: int) -> None:  # moe.rs:192-210
        while self.resident_bytes + size > self.capacity_bytes and self.order:
            if self.evict_lru() is None:
                break
        if key in self.sizes:
            self.resident_bytes -= self.sizes.pop(key)
            if key in self.order:
                self.order.remove(key)
        self.sizes[key] = size
        self.resident_bytes += size
        self.pinned_bytes += size
        self.pinned.add(key)
        self.order.append(key)

    def clear(self) -> None:  # moe.rs:212-218
        self.sizes.clear()
        self.order.clear()
        self.pinned.clear()
        self.resident_bytes = 0
        self.pinned_bytes = 0

    def reset_counters(self) -> None:  # moe.rs:221-226
        for c in COUNTERS:
            setattr(self, c, 0)

    def counters(self) -> dict:
        d = {c: getattr(self, c) for c in COUNTERS}
        d.update(capacity_bytes=self.capacity_bytes, resident_bytes=self.resident_bytes,
                 pinned_bytes=self.pinned_bytes)
        return d


def execute_accounting(cache, fmt: int, tensor_lens, selected, layer_id: int) -> dict:
    """Byte accounting of one executor call.

    tensor_lens[e]: lengths of expert e's tensors in load order: (gate, up, down) for the
    block formats (moe.rs:458-583), (gate_w, gate_s, up_w, up_s, down_w, down_s) for FP4
    (moe.rs:1010-1090). Returns the MoeTelemetry byte fields; mutates `cache`."""
    kinds = (GATE, UP, DOWN) if fmt != FP4 else (GATE_WEIGHT, GATE_SCALE, UP_WEIGHT, UP_SCALE,
                                                  DOWN_WEIGHT, DOWN_SCALE)
    w_loaded = w_reused = s_loaded = s_reused = 0
    logical = 0
    per_kind = [0, 0, 0]
    for e, _w in selected:
        lens = tensor_lens[e]
        expert_bytes = sum(lens)
        logical += expert_bytes
        if fmt != FP4:
            per_kind = [per_kind[0] + lens[0], per_kind[1] + lens[1], per_kind[2] + lens[2]]
        else:
            per_kind = [per_kind[0] + lens[0] + lens[1], per_kind[1] + lens[2] + lens[3],
                        per_kind[2] + lens[4] + lens[5]]
        bypass = False
        if cache is not None and expert_bytes > cache.capacity_bytes:
            if cache.bypass_oversized_experts:
                bypass = True
                cache.oversized_expert_bypass_count += 1
            else:
                cache.self_eviction_risk_count += 1
        for kind, n in zip(kinds, lens):
            is_scale = kind in SCALE_KINDS
            key = (layer_id, e, kind, fmt)
            if bypass:
                cache.cache_insert_attempt_count += 1
                cache.cache_insert_bypass_count += 1
                hit = False
            elif cache is not None:
                hit = cache.get(key)
                if not hit:
                    cache.insert(key, n)
            else:
                hit = False
            if hit:
                if is_scale:
                    s_reused += n
                else:
                    w_reused += n
            elif is_scale:
                s_loaded += n
            else:
                w_loaded += n
    return {
        "selected_expert_count": len(selected),
        "logical_expert_bytes_requested": logical,
        "actual_expert_bytes_loaded": w_loaded + s_loaded,
        "resident_cache_bytes_reused": w_reused + s_reused,
        "weight_bytes_loaded": w_loaded, "weight_bytes_reused": w_reused,
        "scale_bytes_loaded": s_loaded, "scale_bytes_reused": s_reused,
        "bytes_by_tensor_kind_gate": per_kind[0], "bytes_by_tensor_kind_up": per_kind[1],
        "bytes_by_tensor_kind_down": per_kind[2],
    }
