"""CPU oracle of DELTA's selective-KV decode path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this package, and only as the checker / the timed CPU baseline; the product
path (delta_amd/) never imports it.
"""
