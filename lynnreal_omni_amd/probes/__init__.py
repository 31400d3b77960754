"""Stand-alone hardware probes used to bound the kernels' rooflines (not part of the path)."""
