"""w8 symmetric per-group weight format (reference: ``src/lemoq/quant``)."""
