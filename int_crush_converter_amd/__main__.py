"""``python -m int_crush_converter_amd`` (same flags as ``python -m converter``)."""
from .cli import main

main()
