"""Self-drafting readers of the route n-gram memory on MI355X: the GPU drafter (the drafter API
of ``drafting/cpu_drafter.py``), draft-tree structure, verification gather and acceptance
(``drafting/tree.py``), and the drafter bundle format (``drafting/export_drafter.py``)."""
