"""Tree descriptor handed to the tree planner (src/beam_engine/kv_tree_node.py:3-19)."""


class KVTreeNode:
    """parent: parent id (-1 for a root); seqlen: tokens from the root through
    this node (cumulative); requests: candidate indices whose path uses it."""

    __slots__ = ("parent", "id", "seqlen", "num_children", "requests")

    def __init__(self):
        self.parent: int = -1
        self.id: int = 0
        self.seqlen: int = 0
        self.num_children: int = 0
        self.requests: list = []

    def __repr__(self):
        return (f"KVTreeNode(id={self.id}, parent={self.parent}, seqlen={self.seqlen}, "
                f"children={self.num_children}, requests={self.requests})")
