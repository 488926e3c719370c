"""Where the /dev/shm handoff lives (the reference's SHM_ROOT, paths.py:18-20).

Prefill and decode processes on one node must agree on this directory.
"""
import os
from pathlib import Path

SHM_ROOT = Path(os.environ.get("PD_SHM_ROOT", "/dev/shm/rngd_kv_cluster"))
