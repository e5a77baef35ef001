"""Module logger (the reference uses loguru; the standard library serves here)."""
import logging

logger = logging.getLogger("dfsattn_amd")
if not logger.handlers:
    _h = logging.StreamHandler()
    _h.setFormatter(logging.Formatter("%(asctime)s %(levelname)s dfsattn_amd: %(message)s"))
    logger.addHandler(_h)
    logger.setLevel(logging.INFO)
