"""Anvil's MI355X backend: kernel IR -> one .hip file -> a gfx950 shared library."""
__version__ = "0.1.0"
