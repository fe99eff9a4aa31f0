"""Codec core: E8 quantizer, symbolisation, compact storage, rANS, dequant, RHT."""
