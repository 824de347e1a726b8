"""Launch runtime: `Launcher` / `bind` (launcher.py) and the MI355X library binding (mi355x.py)."""
