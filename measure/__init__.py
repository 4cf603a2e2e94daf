"""Measurement aids beside the product library: the streaming-read probe
(libalveare_probe.so, the practical HBM ceiling per launch) and the rocprofv3
summariser that turns kernel traces and counters into the profiles/ tables."""
