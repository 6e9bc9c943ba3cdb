"""Serving the n-gram tables: the serving row layout and host-RAM row providers (drop-in for the
reference's ``serving/layout.py`` and ``serving/prefetch.py``)."""
