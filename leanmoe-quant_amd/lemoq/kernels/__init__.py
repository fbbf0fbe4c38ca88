"""Operator surface of the decode hot path (names follow the reference's
``src/lemoq/kernels``).  Import the submodules directly, e.g.
``from lemoq.kernels.moe_grouped_quant import grouped_moe_forward_quant``."""
