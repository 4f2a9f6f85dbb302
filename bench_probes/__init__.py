"""Measurement probes for bench.py: the streaming-ceiling library
(``libms_hbm_probe.so``) and the K3 placement runs.  Not part of the
minispeed_amd package; nothing on the boundary path imports this."""
