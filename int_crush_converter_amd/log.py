"""Package logger.

The logger is named ``"converter"`` like the reference's (``converter/log.py:18-21``)
so that an application that configured handlers for the reference keeps
receiving the same records.  A ``NullHandler`` keeps library use silent.
"""

import logging

logger = logging.getLogger("converter")
logger.addHandler(logging.NullHandler())
