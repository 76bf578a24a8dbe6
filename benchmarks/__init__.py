"""Benchmarks, probes and sweeps behind the committed profiles (not part of
the zinc_amd product package)."""
