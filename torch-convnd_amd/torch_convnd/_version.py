"""Package version: the reference API level plus this build's local tag."""

__version__ = "0.5.0+gfx950"
