"""Checkpoint formats of the expert banks (reference ``checkpoint/``)."""

from .ftw import FTWReader, FTWWriter, is_ftw_checkpoint, load_ftw_banks, save_ftw_banks

__all__ = ["FTWReader", "FTWWriter", "is_ftw_checkpoint", "load_ftw_banks", "save_ftw_banks"]
