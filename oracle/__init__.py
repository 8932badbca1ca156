"""CPU oracle for the megakernel VM -- TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker / CPU reference; never by the product package.
"""
