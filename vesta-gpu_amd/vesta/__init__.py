"""Vesta: a four-form language (law, fold, fork, residue) and a compiler that
lowers a program to one persistent HIP kernel per step on MI355X (gfx950).

    vesta.interp   lexer and parser of the language (the frontend)
    vesta.lower    program -> HIP C++ for one persistent kernel
    vesta.launch   hipRTC compile and cooperative launch through libvesta_hip.so
    vesta.gpt2     GPT-2 decode on the GPU (VestaGPT2)
    vesta.weights  seeded random-init GPT-2 weights with Hugging Face names

Mirrors the reference package layout (reference vesta/__init__.py:1-12).
"""
from pathlib import Path

__version__ = '0.1.0'
PROGRAMS = Path(__file__).resolve().parent / 'programs'
