"""gfx950 mirror of the reference's ``kairyu.quant`` package."""

from kairyu_amd.quant.linear import linear_factory, make_linear

__all__ = ["linear_factory", "make_linear"]
