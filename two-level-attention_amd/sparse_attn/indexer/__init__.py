"""Indexer configuration (TIA base + NFA two-level selector)."""
from .base import Indexer
from .tia_indexer import TIAIndexer
from .nfa_indexer import NFAIndexer

indexer_type_dict = {
    'tia': TIAIndexer,
    'nfa': NFAIndexer,
}
