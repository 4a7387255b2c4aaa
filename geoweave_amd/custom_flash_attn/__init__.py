"""Custom flash attention operators (gfx950). Mirrors the reference package
``easyvolcap/utils/custom_flash_attn``; the operators live in ``sparse_index_flash_attn``."""
