"""CPU oracle for the Qwen3-TTS token loop.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the cpu_baseline
leg of bench.py may import this package, and only as the checker (or the timed CPU
baseline), never as part of the product path.
"""
