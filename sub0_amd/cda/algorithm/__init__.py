"""Host-side tables of the CDA algorithm (drop-in for ``cda/algorithm``)."""
