"""MI355X (gfx950) implementation of Pyramid Forcing's per-step pyramid
KV-cache path behind the reference's ``pyramidkv`` API."""
