"""Radix-tree prefix cache over paged KV blocks.

Drop-in for the reference's RadixCache (python_runtime/engine/cache/
radix_cache.py:43-247): the same node structure (token run, children keyed
by first token, physical blocks, reference count), the same block
accounting and results, over any block manager with `block_size`,
`increment_ref_count` and `free_block` -- in this build
python_runtime.engine.block_manager.BlockManager.

Block accounting, kept identical because callers depend on it:
- match_prefix returns the blocks of every fully matched node plus, when
  the query ends inside a node, that node's first ceil(matched / block_size)
  blocks -- so a partially filled last block can be returned and shared.
  BlockManager.prepare_writes copies such a block before anyone writes into
  it (copy-on-write), which the reference leaves to the caller.
- insert walks matching nodes, advancing through the new sequence's blocks
  by each fully matched node's block count; a partial match splits the node
  (the shared head keeps the first ceil(common / block_size) blocks, the
  tail the rest); the unmatched remainder becomes a leaf owning the
  remaining new blocks, each gaining one block-manager reference.
- evict frees, depth first and children before parents, nodes whose
  reference count is 0 until the target is met.
"""

from __future__ import annotations

from typing import Any


class RadixTreeNode:
    """A run of tokens, its children (by first token) and its KV blocks."""

    __slots__ = ("token_ids", "children", "kv_blocks", "ref_count")

    def __init__(self, token_ids: tuple[int, ...]) -> None:
        self.token_ids: tuple[int, ...] = token_ids
        self.children: dict[int, RadixTreeNode] = {}
        self.kv_blocks: list[int] = []
        self.ref_count: int = 0

    def __repr__(self) -> str:
        return (f"RadixTreeNode(tokens={self.token_ids[:8]}..., children={len(self.children)}, "
                f"blocks={len(self.kv_blocks)}, ref={self.ref_count})")


def _common_prefix_len(a: list[int] | tuple[int, ...], b: tuple[int, ...]) -> int:
    n = min(len(a), len(b))
    i = 0
    while i < n and a[i] == b[i]:
        i += 1
    return i


def _ceil_div(a: int, b: int) -> int:
    return -(-a // b)


class RadixCache:
    """Prefix cache keyed by token sequences, holding block references."""

    def __init__(self, block_manager: Any) -> None:
        self._bm = block_manager
        self.root = RadixTreeNode(())

    def match_prefix(self, token_ids: list[int]) -> tuple[list[int], int]:
        """(blocks, tokens) of the longest cached prefix of token_ids."""
        blocks: list[int] = []
        matched = 0
        node, rest = self.root, list(token_ids)
        while rest:
            child = node.children.get(rest[0])
            if child is None:
                break
            common = _common_prefix_len(rest, child.token_ids)
            if common < len(child.token_ids):
                blocks += child.kv_blocks[: _ceil_div(common, self._bm.block_size)]
                matched += common
                break
            blocks += child.kv_blocks
            matched += common
            rest = rest[common:]
            node = child
        return blocks, matched

    def insert(self, token_ids: list[int], kv_blocks: list[int]) -> None:
        """Adds a token sequence whose KV sits in kv_blocks."""
        if not token_ids:
            return
        node, rest, used = self.root, list(token_ids), 0
        while rest:
            child = node.children.get(rest[0])
            common = 0 if child is None else _common_prefix_len(rest, child.token_ids)
            if child is None or common == 0:
                self._add_leaf(node, tuple(rest), kv_blocks[used:])
                return
            if common < len(child.token_ids):
                # split: a head node for the shared tokens, the old node below it
                keep = _ceil_div(common, self._bm.block_size)
                head = RadixTreeNode(child.token_ids[:common])
                head.kv_blocks = child.kv_blocks[:keep]
                head.ref_count = child.ref_count
                child.token_ids = child.token_ids[common:]
                child.kv_blocks = child.kv_blocks[keep:]
                head.children[child.token_ids[0]] = child
                node.children[rest[0]] = head
                rest = rest[common:]
                node = head
            else:
                rest = rest[common:]
                used += len(child.kv_blocks)
                node = child

    def evict(self, target_blocks: int) -> int:
        """Frees blocks of unreferenced nodes, leaves first, until
        target_blocks are freed; returns the number freed."""
        if target_blocks <= 0:
            return 0
        freed = 0

        def visit(node: RadixTreeNode, parent: RadixTreeNode, key: int) -> int:
            nonlocal freed
            here = 0
            for k, c in list(node.children.items()):
                here += visit(c, node, k)
            if here >= target_blocks - freed:
                return here
            if node.ref_count == 0:
                for bid in node.kv_blocks:
                    self._bm.free_block(bid)
                    freed += 1
                del parent.children[key]
                here += len(node.kv_blocks)
            return here

        for k, c in list(self.root.children.items()):
            visit(c, self.root, k)
            if freed >= target_blocks:
                break
        return freed

    def _add_leaf(self, parent: RadixTreeNode, token_ids: tuple[int, ...], kv_blocks: list[int]) -> None:
        node = RadixTreeNode(token_ids)
        node.kv_blocks = list(kv_blocks)
        node.ref_count = 1
        for bid in node.kv_blocks:
            self._bm.increment_ref_count(bid)
        parent.children[token_ids[0]] = node


__all__ = ["RadixCache", "RadixTreeNode"]
