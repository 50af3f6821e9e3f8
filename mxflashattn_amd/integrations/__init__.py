"""Framework adapters for the MI355X decode path."""
