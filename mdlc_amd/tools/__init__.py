"""Model builders, the compile CLI and benchmark helpers."""
