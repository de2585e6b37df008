"""Harness utilities: timing/tuning, workload arithmetic, model configs, CSV IO, provenance."""
