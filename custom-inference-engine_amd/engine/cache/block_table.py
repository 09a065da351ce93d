"""Per-sequence logical -> physical block map.

Same fields and methods as the reference's ``engine/cache/block_table.py:7-36``:
``block_size``, ``blocks`` (physical ids in logical order), ``length``
(tokens written); token ``pos`` lives in ``blocks[pos // block_size]`` at
offset ``pos % block_size``.
"""

from __future__ import annotations

from dataclasses import dataclass, field


@dataclass
class BlockTable:
    block_size: int
    blocks: list[int] = field(default_factory=list)
    length: int = 0

    def num_blocks_needed(self, new_length: int) -> int:
        """Blocks that hold ``new_length`` tokens (ceil division)."""
        return -(-new_length // self.block_size)

    def logical_to_physical(self, pos: int) -> tuple[int, int]:
        q, r = divmod(pos, self.block_size)
        return self.blocks[q], r

    def clone(self) -> "BlockTable":
        """Independent copy of the map (the K/V data itself is not copied)."""
        return BlockTable(self.block_size, self.blocks.copy(), self.length)

    def truncate(self, new_length: int) -> None:
        """Shorten to ``new_length`` tokens, dropping the blocks no longer
        needed from the map (the caller returns them to its free list)."""
        assert new_length <= self.length
        self.length = new_length
        self.blocks[self.num_blocks_needed(new_length):] = []
