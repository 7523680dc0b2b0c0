"""Element-wise model of the reference's code-storage rules on a bit-width change, for tests.

/root/reference/CUDA/stquant_opt_simple.py moves a tensor's codes in two stages around the
kernel:
- before the kernel (:140-173), to the width's kernel storage:
  - packed nibbles are split into m = (b & 15) - 8 and v = b >> 4 (int8 / uint8);
  - above 16 bits everything is widened to int32 / uint32;
  - for 9..16 bits int32 codes are clamped to the int16 / uint16 ranges, and narrower codes
    are widened;
  - up to 8 bits int16 / int32 codes are clamped to the int8 / uint8 ranges;
- after the kernel (:175-210), at 4 bits only, the int8 / uint8 codes are packed as
  clamp(m + 8, 0, 15) | clamp(v, 0, 15) << 4.

Here these rules act on Python integers one element at a time, stated from that description;
the product's ``mdq_hip.storage`` states the same moves as one decode -> clamp -> encode map, and
the tests compare the two."""
import numpy as np

P4, S8, S16, S32 = 0, 1, 2, 3
RANGES = {S8: ((-128, 127), 255), S16: ((-32768, 32767), 65535), S32: ((-2 ** 31, 2 ** 31 - 1), 2 ** 32 - 1)}


def _clamp(x, lo, hi):
    return lo if x < lo else hi if x > hi else x


def before_kernel(src, m, v, bits):
    """(layout, m, v) of one element after the pre-kernel stage.  For P4, ``m`` is the byte and
    ``v`` is ignored."""
    if src == P4:
        src, m, v = S8, (m & 15) - 8, m >> 4
    if bits >= 32:
        return S32, m, v
    if bits > 8:
        if src == S32:
            (lo, hi), vhi = RANGES[S16]
            m, v = _clamp(m, lo, hi), _clamp(v, 0, vhi)
        return S16, m, v
    if src in (S16, S32):
        (lo, hi), vhi = RANGES[S8]
        m, v = _clamp(m, lo, hi), _clamp(v, 0, vhi)
    return S8, m, v


def after_kernel(layout, m, v, bits):
    """(layout, m, v) after the post-kernel stage (for P4, ``m`` is the byte and ``v`` None)."""
    if bits == 4 and layout == S8:
        return P4, _clamp(m + 8, 0, 15) | (_clamp(v, 0, 15) << 4), None
    return layout, m, v


def model_arrays(fn, src, m, v, bits):
    """Apply ``fn`` to numpy int64 arrays; returns (layout, m array, v array or None)."""
    out = [fn(src, int(a), int(b), bits) for a, b in zip(m, v)]
    lay = out[0][0] if out else None
    mm = np.array([o[1] for o in out], dtype=np.int64)
    vv = None if lay == P4 else np.array([o[2] for o in out], dtype=np.int64)
    return lay, mm, vv
