"""lemoq (MI355X build) — the batch-1 OLMoE w8a16 decode path of LeanMoE-Quant on
hand-written HIP kernels for gfx950.

The public operator names and signatures follow the reference package
``lemoq`` (``src/lemoq/kernels/*.py``, ``src/lemoq/quant/*.py``) so callers of the
decode hot path can switch over; the kernels behind them are this package's own
HIP code in ``csrc/`` reached through the C-ABI in ``include/lemoq_hip.h``.
"""

__version__ = "0.1.0"
