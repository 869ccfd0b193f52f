"""Base indexer: holds the parsed flags (reference indexer/base.py:8-11)."""


class Indexer:
    def __init__(self, args) -> None:
        self.args = args

    def get_block_size(self):
        return 1

    def clear(self):
        pass
