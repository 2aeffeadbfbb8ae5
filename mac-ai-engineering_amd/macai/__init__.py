"""macai for MI355X: the chunked gated delta rule (the reference's macai.gated_delta hot path) on gfx950."""
__version__ = "0.2.0+mi355x"
