"""CPU restatement of the reference's MoE expert path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or the timed CPU baseline);
product code never imports it.
"""
