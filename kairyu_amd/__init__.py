"""kairyu_amd: the quantized-linear hot path of Kairyu, rebuilt for MI355X (gfx950).

Host code mirrors the reference's ``kairyu.quant`` interface; device work runs
in hand-written HIP kernels behind the C ABI of ``include/kairyu_quant.h``.
"""

__version__ = "0.1.0"
