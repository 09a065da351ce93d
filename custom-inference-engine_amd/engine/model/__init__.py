"""Model-side use of the attention path (the attention section of the
reference's ``engine/model/block.py``)."""

from engine.model.block import attention_section, attention_section_rows  # noqa: F401
