"""Model-level pieces of the INT8-tier hot path (mirror of reference ksdraft/model): the
Rosa mixer, whose hard match and credits run in libksdraft_amd.so."""
