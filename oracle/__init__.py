"""Test infrastructure: CPU oracle for the Lizard attention hot path.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``; never by the product package.
"""
