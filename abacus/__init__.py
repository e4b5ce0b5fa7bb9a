"""Drop-in namespace with abacus's module paths.

Each module re-exports the MI355X implementation from ``abacus_amd`` under the
name the reference uses, so code written against abacus (e.g. its
transformer_block.py and tests/test_moe.py imports) resolves to the HIP path.
"""
