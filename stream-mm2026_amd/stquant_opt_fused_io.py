"""MDQAdamWSimpleFusedIO -- drop-in for /root/reference/CUDA/stquant_opt_fused_io.py.

A tensor whose codes already rest in the layout of its ``current_bit`` (packed nibbles at 4
bits, int8/uint8 at 8, int16/uint16 at 16, int32/uint32 at 32) goes straight to the fused
kernel.  Any other tensor falls back to MDQAdamWSimple's route.  The fallback increments
``state['step']`` twice, as in the reference (:44 then stquant_opt_simple.py:236).  The
timing dict reports the fast-path and fallback counts and the fast-path ratio.
"""
from __future__ import annotations

from stquant_opt_simple import MDQAdamWSimple


class MDQAdamWSimpleFusedIO(MDQAdamWSimple):
    """MDQ Simple + the no-pack/unpack fast path when the storage already fits."""

    def _begin_update(self, p, group) -> bool:
        # stquant_opt_fused_io.py:39-54: count the path, and on a fallback let the Simple
        # route increment the step a second time
        state = self.state[p]
        state["step"] += 1
        lt = self.last_step_timings
        if self._storage_matches_bits(state, int(state["current_bit"])):
            lt["mdq_fused_io_fast_path_params"] += 1
            return False
        lt["mdq_fused_io_fallback_params"] += 1
        return super()._begin_update(p, group)

    def _count_steady_params(self, n: int) -> None:
        # a steady step only runs tensors whose storage already matches
        self.last_step_timings["mdq_fused_io_fast_path_params"] = n

    def _finalize_step_timings(self, profile_device):
        # stquant_opt_fused_io.py:86-93
        super()._finalize_step_timings(profile_device)
        lt = self.last_step_timings
        fast, total = lt["mdq_fused_io_fast_path_params"], lt["mdq_fused_io_fast_path_params"] + lt[
            "mdq_fused_io_fallback_params"]
        lt["mdq_fused_io_fast_path_ratio"] = fast / total if total > 0 else 0.0
