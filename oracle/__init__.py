"""CPU oracle for TinyTensor scaled dot-product attention.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
package; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker or as
the timed CPU baseline.
"""
