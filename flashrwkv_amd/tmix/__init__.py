"""TimeMix operators (WKV7 only in this build)."""
