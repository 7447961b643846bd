"""Test infrastructure: CPU restatement of the reference chunked GatedDeltaNet forward.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
package, as the checker.  The product path (kairos-sensenova_amd) never does.
"""
