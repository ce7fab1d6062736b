"""Runtime: hipRTC + HIP module boundary (hip.py), JIT (jit.py), autotuning."""
