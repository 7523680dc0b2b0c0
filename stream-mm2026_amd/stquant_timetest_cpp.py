"""Drop-in for the reference's compiled module ``stquant_timetest_cpp``.

The reference builds it from /root/reference/CUDA/stquant_core.cpp:9-15 (pybind11)
over launch_fused_mdq_adamw (/root/reference/CUDA/stquant_kernel.cu:414-465).  Here
the same function calls the C ABI of ``libstquant_hip.so`` (gfx950 HIP kernels).
"""
from mdq_hip import fused_step as _fused_step


def fused_mdq_adamw(p, grad, exp_avg, exp_avg_sq, scale_m, scale_v, v_min,
                    beta1, beta2, lr, weight_decay, eps, step, bits, block_size,
                    profile_cycles=None, *, rounding="nearest", seed=0, tensor_id=0):
    """MDQ AdamW fused update, in place, asynchronous on the current stream.

    Arguments as the reference's (stquant_core.cpp:3-7).  ``profile_cycles``:
    optional device int64[5] receiving += clock64 cycles of the dequant /
    adam_mv / scale_reduce / quant / update_p phases.  Keyword-only
    extensions: ``rounding`` ('nearest' | 'stochastic'), ``seed`` and
    ``tensor_id`` (the stochastic-rounding stream).
    """
    _fused_step(p, grad, exp_avg, exp_avg_sq, scale_m, scale_v, v_min,
                beta1, beta2, lr, weight_decay, eps, step, bits, block_size, profile_cycles,
                rounding=rounding, seed=seed, tensor_id=tensor_id)
