"""MDQAdamWSimpleFusedIO -- drop-in for /root/reference/CUDA/stquant_opt_fused_io.py.

When the code storage already matches ``current_bit`` (packed nibbles at 4
bits, int8/uint8 at 8, int16/uint16 at 16, int32/uint32 at 32) the tensor goes
straight to the fused kernel with no pack/unpack; otherwise it falls back to
MDQAdamWSimple's route.  As in the reference (:44 then stquant_opt_simple.py:236)
the fallback increments ``state['step']`` twice.  Fast-path / fallback counts
and the fast-path ratio are reported in the timing dict.
"""
from __future__ import annotations

from stquant_opt_simple import MDQAdamWSimple


class MDQAdamWSimpleFusedIO(MDQAdamWSimple):
    """MDQ Simple + the no-pack/unpack fast path when the storage already fits."""

    def _prepare_update(self, p, group):
        # stquant_opt_fused_io.py:39-54
        state = self.state[p]
        bits = int(state["current_bit"])
        state["step"] += 1
        lt = self.last_step_timings
        if not self._storage_matches_bits(state, bits):
            lt["mdq_fused_io_fallback_params"] = lt.get("mdq_fused_io_fallback_params", 0) + 1
            return super()._prepare_update(p, group)
        lt["mdq_fused_io_fast_path_params"] = lt.get("mdq_fused_io_fast_path_params", 0) + 1
        return False

    def _count_steady_params(self, n: int) -> None:
        # a steady step only runs tensors whose storage already matches
        self.last_step_timings["mdq_fused_io_fast_path_params"] = n

    def _finalize_step_timings(self, profile_device):
        # stquant_opt_fused_io.py:86-93
        super()._finalize_step_timings(profile_device)
        fast_n = int(self.last_step_timings.get("mdq_fused_io_fast_path_params", 0))
        fall_n = int(self.last_step_timings.get("mdq_fused_io_fallback_params", 0))
        total = fast_n + fall_n
        self.last_step_timings["mdq_fused_io_fast_path_ratio"] = (fast_n / total) if total > 0 else 0.0
